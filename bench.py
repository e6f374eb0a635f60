"""Benchmark of the int8 hot path on one MI355X, with its roofline and the host baseline.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload decode|gemv]

Prints ONE JSON line.

``decode`` (default): a random-init Qwen2.5-0.5B-shaped
model (24 layers, hidden 896, 14/2 heads of 64, MLP 4864, vocab 151936, tied
float32 LM head), all 168 projections per-row int8 with per-token int8
activations; a 128-token prompt of uniform-random ids, then 256 greedy tokens
(past to 384) whatever ``--steps`` is. A step is one decode token: one replay
of the captured decode step (every layer, the LM head, the argmax, the
feedback of the token). The timed region is the last K of the 255 replays
(default all 255), ending at past 383, bracketed by HIP events on the library
stream; the mean over all 255 is reported under ``config.all_replays``. Each
kernel group of the step (qkv, attention, o, gate/up, down, LM head) is then
timed live, and the single kernel with the most time a step is the line's
``roofline`` (attention's two kernels, timed together, are reported beside it
under ``roofline.attention``). The host C
model (oracle/nc_model.c) decodes the same prompt on this machine's cores in
the same run; all 256 of its tokens must equal the GPU's, and a thread sweep
of its decode steps is the CPU baseline, with config 1's GEMV on the host
(thread sweep, GB/s) beside it.

``gemv``: the decode projection [1,896] x [4864,896]^T,
weights rotated through 128 device copies (560 MB, past the 256 MB Infinity
Cache) in one stacked launch, under each GEMV launch shape (schedules 0..7,
each checked bit for bit): the fastest is the streaming rate, reported with
its schedule and every shape's rate; one launch alone (the default shape) is
reported too. Also measured in the default run and reported under "gemv".

The default run also measures, on the same model's weights, and reports under
``config.blocks``: config 2 (the fused rms_norm -> int8 row kernel at 1, 64
and 512 rows), config 3 (one decoder block's decode step at past 512, per
block over all 24) and config 4 (one block's prefill of 512 tokens, per
block, and its four MFMA GEMM shapes alone, with MFMA utilisation against the
5.0 POP/s dense int8 peak).

Roofline numerators are algorithmic bytes:
  GEMV:    N*K + 4N + M*K + 4M + 4MN = 4,397,956 B per [1,896]x[4864,896]^T.
  LM head: 4*V*H (float32 table) + 4*H (x) + 8 (argmax key) = 544,542,216 B per step.
  Block decode (past 512): 15,507,456 B.  GEMM: M*K + N*K + 4MN + 4M + 4N.

Before anything else the run copies 256 MiB device to device once
(``__amd_rocclr_copyBuffer``): a copy of known size whose FETCH_SIZE and
WRITE_SIZE calibrate the profiler's byte counters.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

import numpy as np

HBM_PEAK_GBPS = 8000.0
N, K, M = 4864, 896, 1
COPIES = 128
GEMV_SCHEDULES = range(8)      # 0: the library's default; 1..7: the GEMV's launch shapes
PROMPT, NEW_TOKENS = 128, 256
CALIBRATION_BYTES = 256 * 2**20


# Each decode-step kernel group's kernel symbol (as a rocprofv3 kernel trace names it).
KERNEL_SYMBOLS = {"qkv": "gemv_decode<896, 0, 0, 8, 1, 16>",
                  "attention": "attention_decode_chunks<64, true> + attention_combine<64, 8>",
                  "o": "gemv_decode<896, 1, 1, 8, 1, 16>", "gate/up": "gemv_decode<896, 0, 2, 8, 1, 16>",
                  "down": "gemv_decode<4864, 1, 1, 64, 4, 4>", "lm head": "lm_head_ring<896, 24>"}


def gemv_bytes(m: int, n: int, k: int) -> int:
    return n * k + 4 * n + m * k + 4 * m + 4 * m * n


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


TRAFFIC = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "traffic.json")


def measured_traffic(kernel: str) -> int | None:
    """HBM bytes per launch of `kernel` from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE
    passes (profiles/traffic.json, counters calibrated on a copy of known size), or None."""
    try:
        with open(TRAFFIC, encoding="utf-8") as f:
            return int(json.load(f)["kernels"][kernel]["traffic_bytes"])
    except (OSError, KeyError, ValueError):
        return None


# -- config 1: the decode GEMV -----------------------------------------------------


def gpu_gemv(steps: int, warmup: int, seed: int = 0) -> dict:
    from nanocompile_amd import hip, kernels
    from nanocompile_amd.hip import DeviceArray, Event

    hip.init(0)
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    x = rng.standard_normal((M, K)).astype(np.float32)
    q1, s1 = kernels.quantize_int8(w)
    xq1, xs1 = kernels.quantize_token(x)
    q = DeviceArray((COPIES, N, K), np.int8)
    ws = DeviceArray((COPIES, N), np.float32)
    xq = DeviceArray((COPIES, M, K), np.int8)
    xs = DeviceArray((COPIES, M), np.float32)
    lib = hip.load()
    for c in range(COPIES):
        lib.nc_memcpy_d2d(q.ptr + c * N * K, q1.ptr, N * K)
        lib.nc_memcpy_d2d(ws.ptr + c * N * 4, s1.ptr, N * 4)
        lib.nc_memcpy_d2d(xq.ptr + c * M * K, xq1.ptr, M * K)
        lib.nc_memcpy_d2d(xs.ptr + c * M * 4, xs1.ptr, M * 4)
    hip.sync()
    y = DeviceArray((COPIES, M, N), np.float32)

    single = kernels.matmul_i8_token(xq1, xs1, q1, s1).numpy()
    kernels.matmul_i8_token_stacked(xq, xs, q, ws, out=y)
    stacked = y.numpy()
    if not all(np.array_equal(stacked[c], single) for c in range(COPIES)):
        raise RuntimeError("stacked GEMV differs from the single GEMV")

    out1 = DeviceArray((M, N), np.float32)
    args_single = [[out1, xq.ptr + c * M * K, xs.ptr + c * M * 4, q.ptr + c * N * K, ws.ptr + c * N * 4]
                   for c in range(COPIES)]
    for a in args_single[:8]:
        hip.call("nc_matmul_i8_token", a, [M, N, K, 0])
    hip.sync()
    starts, stops = [Event() for _ in range(COPIES)], [Event() for _ in range(COPIES)]
    for c in range(COPIES):
        starts[c].record()
        hip.call("nc_matmul_i8_token", args_single[c], [M, N, K, 0])
        stops[c].record()
    hip.sync()
    single_us = statistics.median(starts[c].elapsed_ms(stops[c]) * 1e3 for c in range(COPIES))

    # The stacked stream under each GEMV launch shape (schedule 0: the library's
    # default, tuned for one latency-bound launch; 1..7: lanes per row x waves,
    # nc_schedule_info), each checked bit for bit first: the fastest is the
    # kernel's streaming rate, reported with its schedule and the default's.
    stacked_args = [y, xq, xs, q, ws]
    per_launch_bytes = gemv_bytes(M, N, K) * COPIES
    by_schedule = {}
    for sched in GEMV_SCHEDULES:
        hip.call("nc_matmul_i8_token_stacked", stacked_args, [COPIES, M, N, K, sched])
        out = y.numpy()
        if not all(np.array_equal(out[c], single) for c in (0, COPIES // 2, COPIES - 1)):
            raise RuntimeError(f"stacked GEMV schedule {sched} differs from the single GEMV")
        for _ in range(warmup):
            hip.call("nc_matmul_i8_token_stacked", stacked_args, [COPIES, M, N, K, sched])
        hip.sync()
        ev = [(Event(), Event()) for _ in range(steps)]
        for a, b in ev:
            a.record()
            hip.call("nc_matmul_i8_token_stacked", stacked_args, [COPIES, M, N, K, sched])
            b.record()
        hip.sync()
        by_schedule[sched] = statistics.fmean(a.elapsed_ms(b) for a, b in ev)
    best = min(by_schedule, key=by_schedule.get)
    mean_ms = by_schedule[best]
    shape = hip.schedule_info(best) if best > 0 else None
    lanes, waves = (int(shape["lanes_per_row"]), int(shape["waves"])) if shape else (8, 1)
    return {"stacked_ms": mean_ms, "stacked_gbps": per_launch_bytes / (mean_ms * 1e-3) / 1e9,
            "schedule": best, "lanes_per_row": lanes, "waves": waves,
            "by_schedule_gbps": {str(k): round(per_launch_bytes / (v * 1e-3) / 1e9, 1) for k, v in by_schedule.items()},
            "single_us": single_us, "single_gbps": gemv_bytes(M, N, K) / (single_us * 1e-6) / 1e9,
            "per_launch_bytes": per_launch_bytes}


def cpu_gemv(seconds: float = 6.0, seed: int = 0) -> dict:
    from oracle import build, host
    if not build.LIBRARY.exists():
        build.build()
    rng = np.random.default_rng(seed)
    cores = os.cpu_count() or 1
    copies = 240
    q = rng.integers(-127, 128, (copies, N, K), dtype=np.int8)
    ws = (rng.random((copies, N)) * 1e-3).astype(np.float32)
    xq = rng.integers(-127, 128, (M, K), dtype=np.int8)
    xs = np.ones(M, np.float32)
    counts = sorted({1, 4, 8, 16, min(cores, 64)} & set(range(1, min(cores, 64) + 1)))
    results = {}
    for t in counts:
        host.set_threads(t)
        s1 = host.time_matmul_i8_token(xq, xs, q, ws, 1)
        reps = max(1, int(seconds / len(counts) / max(s1, 1e-6)))
        s = host.time_matmul_i8_token(xq, xs, q, ws, reps)
        results[t] = gemv_bytes(M, N, K) * copies * reps / s / 1e9
    best = max(results, key=results.get)
    return {"gbps": results[best], "threads": best, "by_threads": {str(k): round(v, 2) for k, v in results.items()},
            "isa": host.isa(), "cores": cores}


def cpu_blocks(seconds: float = 12.0, seed: int = 7) -> dict:
    """Configs 2-4 on the host C path (oracle/nc_host.c, oracle/nc_model.c: the build's own C, the
    reference having no per-token int8 mode), on this machine's cores. Config 2: rms_norm -> int8
    of 512 rows (the host row kernel runs on one thread). Configs 3 and 4: one Qwen2.5-0.5B-shaped
    decoder block as a one-layer host model whose tied head has 64 rows (0.2 MB beside the block's
    15 MB), a decode step at past 512 and a 512-token prefill, threads swept."""
    import dataclasses
    from oracle import host
    from oracle.host_model import HostQwen2
    from nanocompile_amd.models.config import QWEN25_05B, random_weights
    cores = os.cpu_count() or 1
    counts = sorted({1, 2, 4, 8, 16, min(cores, 64)} & set(range(1, min(cores, 64) + 1)))
    rng = np.random.default_rng(seed)
    c = QWEN25_05B
    x = rng.standard_normal((512, c.hidden_size)).astype(np.float32)
    x[rng.random(x.shape) < 0.01] *= 20
    gamma = (1 + 0.1 * rng.standard_normal(c.hidden_size)).astype(np.float32)
    rms_by_threads = {}
    for t in counts:                               # config 2's rows spread over the pool, threads swept
        host.set_threads(t)
        host.rms_norm_quant_pool(x, gamma, c.rms_norm_eps)
        t0, reps = time.perf_counter(), 0
        while reps < 3 or time.perf_counter() - t0 < 1.0 / len(counts) + 0.2:
            host.rms_norm_quant_pool(x, gamma, c.rms_norm_eps)
            reps += 1
        rms_by_threads[t] = (time.perf_counter() - t0) / reps * 1e6
    rms_threads = min(rms_by_threads, key=rms_by_threads.get)
    rms_us = rms_by_threads[rms_threads]

    one = dataclasses.replace(c, num_hidden_layers=1, vocab_size=64)
    past = 512
    model = HostQwen2(one, random_weights(one, seed=seed), capacity=past + 8)
    model.kcache[...] = rng.standard_normal(model.kcache.shape).astype(np.float32)
    model.vcache[...] = rng.standard_normal(model.vcache.shape).astype(np.float32)
    prompt = rng.integers(0, one.vocab_size, 512)

    def timed(run, budget: float) -> float:
        run()                                   # the pool's threads up, caches warm
        t, n = time.perf_counter(), 0
        while n < 2 or time.perf_counter() - t < budget:
            run()
            n += 1
        return (time.perf_counter() - t) / n

    decode_us, prefill_us = {}, {}
    for t in counts:
        host.set_threads(t)

        def step():
            model.length = past
            model.forward([7])

        def prompt_pass():
            model.length = 0
            model.forward(prompt)

        decode_us[t] = timed(step, seconds / 3 / len(counts)) * 1e6
        prefill_us[t] = timed(prompt_pass, seconds / 2 / len(counts)) * 1e6
    bd, bp = min(decode_us, key=decode_us.get), min(prefill_us, key=prefill_us.get)
    return {"cores": cores, "isa": host.isa(),
            "rms_norm_quant_512": {"us": round(rms_us, 2), "threads": rms_threads,
                                   "gbps": round(rms_row_bytes(512) / (rms_us * 1e-6) / 1e9, 2),
                                   "by_threads_us": {str(k): round(v, 2) for k, v in rms_by_threads.items()}},
            "block_decode": {"past": past, "us": round(decode_us[bd], 1), "threads": bd,
                             "gbps": round(BLOCK_DECODE_BYTES / (decode_us[bd] * 1e-6) / 1e9, 2),
                             "by_threads_us": {str(k): round(v, 1) for k, v in decode_us.items()}},
            "block_prefill": {"seq": 512, "us": round(prefill_us[bp], 1), "threads": bp,
                              "tok_s": round(512 / (prefill_us[bp] * 1e-6), 1),
                              "by_threads_us": {str(k): round(v, 1) for k, v in prefill_us.items()}},
            "sample": "config 2: 512 rows on the pool, each thread count repeated for a bounded share of a "
                      "second; configs 3 and 4: a one-layer host model "
                      "(the block, a 64-row head), each thread count timed for a bounded share of "
                      f"{seconds:.0f} s"}


# -- configs 2-4: the fused row kernel, one block's decode step, one block's prefill ----------

MFMA_I8_PEAK_TOPS = 5000.0          # MI355X dense int8 MFMA, 5.0 POP/s
BLOCK_DECODE_BYTES = 15_507_456     # int8 W + scales + biases + gammas + KV read (past 512) + KV write + ~10 KB
PREFILL_SHAPES = {"q/o (896,896)": (896, 896), "k/v (128,896)": (128, 896),
                  "gate/up (4864,896)": (4864, 896), "down (896,4864)": (896, 4864)}


def gemm_bytes(m: int, n: int, k: int) -> int:
    """int8 A and B, f32 output, both scale vectors."""
    return m * k + n * k + 4 * m * n + 4 * m + 4 * n


def rms_row_bytes(m: int, k: int = 896) -> int:
    """Read x, write normed, int8 row and scale per row; gamma once."""
    return m * (4 * k + 4 * k + k + 4) + 4 * k


USE_GRAPHS = True     # False under profilers that cannot follow graph launches (--no-graph)


def graph_us(fn, reps: int, rounds: int = 5) -> float:
    """Median over rounds of one captured graph of ``reps`` calls, per call, in microseconds."""
    from nanocompile_amd import hip
    from nanocompile_amd.hip import Event, Graph
    run = lambda: [fn(i) for i in range(reps)]
    launch = Graph.capture(run).launch if USE_GRAPHS else run
    launch()
    hip.sync()
    a, b = Event(), Event()
    samples = []
    for _ in range(rounds):
        a.record()
        launch()
        b.record()
        hip.sync()
        samples.append(a.elapsed_ms(b) * 1e3 / reps)
    return statistics.median(samples)


def generated_config2(cache=None) -> tuple[dict, dict]:
    """Config 2's graph (rms_norm, then one int8 scale per row, in the reference's graph ops) as
    the reference compiles it, recorded as data (tests/golden/programs.json.gz) and generated as
    HIP by codegen_hip: unfused (its lowering with fuse=False, a kernel per operation,
    runtime.py:186) and fused (its fusion pass), each on the default GPU schedules and with each
    kernel's schedule (threads, LDS staging, workgroup items, vector width, unroll) chosen by the
    autotuner on 1, 64 and 512 rows, per token (``cache``: the autotuner's). Both run from the
    program's candidate library, so every kernel in a trace has its own name. Returns
    ({variant: CompiledProgram}, the tuned schedules by variant)."""
    from nanocompile_amd import autotune, lir
    from nanocompile_amd.compiled import CompiledProgram
    golden = Path(__file__).resolve().parent / "tests" / "golden"
    doc = lir.load_programs(golden / "programs.json.gz")
    with np.load(golden / "programs.npz", allow_pickle=False) as arrays:
        recorded = {variant: lir.program_from_json(doc["zoo"]["rms_norm_quant"][key], arrays)
                    for variant, key in (("unfused", "unfused"), ("fused", "program"))}
    generated = {}
    for variant, program in recorded.items():
        library = autotune.CandidateLibrary(program)
        generated[variant] = CompiledProgram(program, autotune.Chosen(library, [0] * len(library.candidates)))
    tuner = autotune.Autotuner(cache=cache, workloads=[(f"m{m}", {"seq": m}, 1.0 / m) for m in (1, 64, 512)])
    tuned_schedules = {}
    for variant, program in recorded.items():
        first = len(tuner.records)
        generated[f"{variant}_tuned"] = CompiledProgram(program, schedule=tuner)
        tuned_schedules[variant] = {f"kernel {r.shape[0]} ({r.op})": {
            "config": r.config, "speedup": round(r.speedup or 1.0, 3)} for r in tuner.records[first:]}
    return generated, tuned_schedules


def generated_kernels(rows: int = 512, reps: int = 20, seed: int = 7) -> dict:
    """Config 2's generated programs (default and tuned) launched eagerly ``reps`` times at
    ``rows`` rows, for a kernel trace; returns each kernel's launcher and schedule by variant."""
    from nanocompile_amd import hip
    generated, tuned = generated_config2(cache=True)
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((rows, 896)).astype(np.float32)
    gamma = (1 + 0.1 * rng.standard_normal(896)).astype(np.float32)
    out = {}
    for variant, program in generated.items():
        launch, _, _ = program.prepare({"x": x}, {"w": gamma})
        for _ in range(reps):
            launch()
        hip.sync()
        out[variant] = [{"launcher": name, "device": "nc_g" + name[4:], "schedule": launch_.describe()}
                        for name, (_, launch_) in zip(program.launcher_names, program.scheduled)]
    return {"rows": rows, "reps": reps, "kernels": out, "tuned": tuned}


def generated_config5(weights: dict, past: int = PROMPT + NEW_TOKENS - 2, seed: int = 3, cache=None,
                      eager: int = 0, seq: int = 1, rounds: int = 5, reps: int = 4) -> dict:
    """Config 5's decode step through the drop-in path: the reference's own compiled program for
    the model (int8 mode, recorded in tests/golden/programs.json.gz; its tokens and logits are
    checked against the reference's in tests/test_config5_generated_gpu.py) generated as HIP by
    codegen_hip, on these weights (the projections quantized per row on the GPU), at one token
    and ``past`` cached positions; default GPU schedules, then each kernel's schedule chosen by
    the autotuner on that step (``cache``: the autotuner's). Graph-replayed, like the hand-written
    step; with ``eager``, each step is then also launched that many times directly (for a kernel
    trace: both run from the program's candidate library, so every kernel has its own name).
    ``seq`` > 1 with ``past`` 0 is a prompt's prefill instead (config 4: 512 tokens)."""
    from nanocompile_amd import autotune, hip, kernels, lir
    from nanocompile_amd.compiled import CompiledProgram
    from nanocompile_amd.models.config import QWEN25_05B as c
    golden = Path(__file__).resolve().parent / "tests" / "golden"
    doc = lir.load_programs(golden / "programs.json.gz")
    with np.load(golden / "programs.npz", allow_pickle=False) as arrays:
        program = lir.program_from_json(doc["config5"]["last"], arrays)
    ref_weights = {}
    for name in program.weights:
        if name.endswith("@int8"):
            w = name.rsplit("@", 1)[0]
            q, scales = kernels.quantize_int8(weights[w])
            ref_weights[name], ref_weights[w + "@scales"] = q.numpy(), scales.numpy()
        elif not name.endswith("@scales"):
            ref_weights[name] = weights[name]
    rng = np.random.default_rng(seed)
    cache_shape = (c.num_hidden_layers, c.num_key_value_heads, past, c.head_dim)
    inputs = {"token_ids": rng.integers(0, c.vocab_size, seq).astype(np.int64),
              "past_keys": rng.standard_normal(cache_shape).astype(np.float32),
              "past_values": rng.standard_normal(cache_shape).astype(np.float32)}
    out = {"program": f"the reference's int8 program: {len(program.kernels)} kernels, {len(program.calls)} launches "
                      f"a step", "seq": seq, "past": past}
    t0 = time.perf_counter()
    tuner = autotune.Autotuner(cache=cache, rounds=rounds, reps=reps, verbose=True,
                               workloads=[("decode" if seq == 1 else "prefill", {"seq": seq, "past": past}, 1.0 / seq)])
    library = autotune.CandidateLibrary(program)
    for label, schedule in (("default", autotune.Chosen(library, [0] * len(program.kernels))), ("tuned", tuner)):
        log(f"generated: config 5's program, {label} schedules")
        compiled = CompiledProgram(program, schedule=schedule)
        launch, _, _ = compiled.prepare(inputs, ref_weights)
        us = graph_us(lambda i, launch=launch: launch(), 1, rounds=5)
        out[label] = {"us_per_step": round(us, 1), "tok_s": round(seq * 1e6 / us, 1)}
        if eager:
            for _ in range(eager):
                launch()
            hip.sync()
            out[label]["kernels"] = [{"device": "nc_g" + name[4:], "schedule": l.describe(),
                                      "packed": any(p.packed for p in k.params)}
                                     for name, (k, l) in zip(compiled.launcher_names, compiled.scheduled)]
        del compiled
    out["tuned"]["schedules"] = {f"kernel {r.shape[0]} ({r.op})": r.config for r in tuner.records if r.winner}
    out["seconds"] = round(time.perf_counter() - t0, 1)
    return out


def block_measurements(model, seed: int = 7) -> dict:
    """Configs 2, 3 and 4 on the decode model's own weights (24 layers, so weights stream as in the model)."""
    from nanocompile_amd import hip
    from nanocompile_amd.hip import DeviceArray, Graph, Event
    from nanocompile_amd.kernels import float_bits

    c = model.config
    H, I, D, L = c.hidden_size, c.intermediate_size, c.head_dim, c.num_hidden_layers
    heads, kv = c.num_attention_heads, c.num_key_value_heads
    eps = float_bits(c.rms_norm_eps)
    rng = np.random.default_rng(seed)
    out: dict = {}

    # config 2: rms_norm -> per-token int8 at M in {1, 64, 512}, one kernel
    gamma = DeviceArray.from_host((1 + 0.1 * rng.standard_normal(H)).astype(np.float32))
    rows = {}
    for m in (1, 64, 512):
        x = rng.standard_normal((m, H)).astype(np.float32)
        x[rng.random(x.shape) < 0.01] *= 20
        xd = DeviceArray.from_host(x)
        normed, xq, xs = DeviceArray((m, H), np.float32), DeviceArray((m, H), np.int8), DeviceArray((m,), np.float32)
        us = graph_us(lambda i: hip.call("nc_rms_norm_quant", [normed, xq, xs, xd, gamma], [m, H, eps]), 32)
        rows[str(m)] = {"us": round(us, 3), "bytes": rms_row_bytes(m, H),
                        "gbps": round(rms_row_bytes(m, H) / (us * 1e-6) / 1e9, 1)}
    # the same rows through the reference's own compilation of config 2's graph
    generated, tuned_schedules = generated_config2()
    gamma_host = gamma.numpy()
    for m in (1, 64, 512):
        x = rng.standard_normal((m, H)).astype(np.float32)
        for variant, program in generated.items():
            launch, _, _ = program.prepare({"x": x}, {"w": gamma_host})
            us = graph_us(lambda i, launch=launch: launch(), 32)
            rows[str(m)][f"generated_{variant}"] = {"us": round(us, 3), "kernels": len(program.program.calls)}
    out["rms_norm_quant"] = {"kernel": "rms_norm_quant (one pass: normed f32, int8 row, scale)", "rows": rows,
                             "generated": "the reference's program for the same graph, lowered to HIP by "
                                          "codegen_hip (unfused: a kernel per operation; fused: its fusion; "
                                          "_tuned: each kernel's GPU schedule chosen by the autotuner)",
                             "tuned_schedules": tuned_schedules}

    # config 3: one decoder block's decode step at past = 512 (all 24 blocks replayed, per block)
    past = 512
    cache = model.new_cache(past + 8)
    kvals = rng.standard_normal((L, kv, past + 8, D)).astype(np.float32)
    cache.keys.upload(kvals)
    cache.values.upload(rng.standard_normal(kvals.shape).astype(np.float32))
    x0 = DeviceArray.from_host(rng.standard_normal((1, H)).astype(np.float32))
    lib = hip.load()

    def decode_layers(_):
        lib.nc_memcpy_d2d(model.x.ptr, x0.ptr, H * 4)      # same residual input every replay
        model._layers(1, past, cache)

    us = graph_us(decode_layers, 1, rounds=9)
    per_block = us / L
    out["block_decode"] = {"past": past, "block_us": round(per_block, 3), "layers_us": round(us, 2),
                           "bytes_per_block": BLOCK_DECODE_BYTES,
                           "gbps": round(BLOCK_DECODE_BYTES / (per_block * 1e-6) / 1e9, 1),
                           "frac": round(BLOCK_DECODE_BYTES / (per_block * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4),
                           "kernels_per_block": 6}

    # config 4: one block's prefill at seq = 512, past = 0 (all 24 blocks, per block), and its GEMMs alone
    m = 512
    if model.max_tokens >= m:
        pcache = model.new_cache(m)
        ids = DeviceArray.from_host(rng.integers(0, c.vocab_size, m).astype(np.int64))

        def prefill_layers(_):
            hip.call("nc_embed", [model.x, model.embed, ids], [m, H, c.vocab_size])
            model._layers(m, 0, pcache)

        us = graph_us(prefill_layers, 1, rounds=5)
        gemms = {}
        for name, (n, k) in PREFILL_SHAPES.items():
            xq = DeviceArray.from_host(rng.integers(-127, 128, (m, k)).astype(np.int8))
            xs = DeviceArray.from_host((rng.random(m) * 0.05).astype(np.float32))
            y = DeviceArray((m, n), np.float32)
            key = {"q/o (896,896)": "o", "k/v (128,896)": "qkv", "gate/up (4864,896)": "gate",
                   "down (896,4864)": "down"}[name]
            offset = 896 * k if key == "qkv" else 0           # the k rows of the fused qkv matrix
            weights = [(model.layers[i][key][0].ptr + offset, model.layers[i][key][1].ptr + offset // k * 4)
                       for i in range(L)]

            def gemm(i, n=n, k=k, xq=xq, xs=xs, y=y, weights=weights):
                q, s = weights[i % L]
                hip.call("nc_matmul_i8_token", [y, xq, xs, q, s, None, None], [m, n, k, 0])

            t = graph_us(gemm, 2 * L)
            ops = 2 * m * n * k
            gemms[name] = {"us": round(t, 3), "tops": round(ops / (t * 1e-6) / 1e12, 1),
                           "mfma_frac": round(ops / (t * 1e-6) / 1e12 / MFMA_I8_PEAK_TOPS, 4),
                           "bytes": gemm_bytes(m, n, k),
                           "hbm_frac": round(gemm_bytes(m, n, k) / (t * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4)}
        out["prefill"] = {"seq": m, "block_us": round(us / L, 2), "layers_us": round(us, 1),
                          "tok_s": round(m / (us * 1e-6), 1), "gemm": gemms,
                          "gemm_kernel": "gemm_i8_mfma (v_mfma_i32_16x16x64_i8, LDS-staged tiles)"}
    return out


def prefill_gemms_vs_library(m: int = 512, copies: int = 8) -> dict:
    """Config 4's int8 GEMMs at M = ``m``: this library's MFMA kernel (its default tile, and every
    tile of its table, with the int32-only epilogue beside the dequantizing one) against the
    vendor library's int8 GEMM (torch._int_mm, int32 out), each graph-replayed over ``copies``
    rotating weight copies. Microseconds a call."""
    import torch
    torch.cuda.init()               # torch's runtime first: it finds no device once ours holds it
    from nanocompile_amd import hip
    from nanocompile_amd.hip import DeviceArray
    hip.init(0)
    rng = np.random.default_rng(0)
    shapes = dict(PREFILL_SHAPES, **{"gate+up as one (9728,896)": (9728, 896)})
    out = {}
    for name, (n, k) in shapes.items():
        xq = DeviceArray.from_host(rng.integers(-127, 128, (m, k)).astype(np.int8))
        xs = DeviceArray.from_host((rng.random(m) * 0.05).astype(np.float32))
        ws = [(DeviceArray.from_host(rng.integers(-127, 128, (n, k)).astype(np.int8)),
               DeviceArray.from_host((rng.random(n) * 0.01).astype(np.float32))) for _ in range(copies)]
        y = DeviceArray((m, n), np.float32)
        acc = DeviceArray((m, n), np.int32)

        def ours(schedule, entry="dequant"):
            if entry == "dequant":
                return graph_us(lambda i: hip.call("nc_matmul_i8_token", [y, xq, xs, ws[i % copies][0],
                                                                          ws[i % copies][1], None, None],
                                                   [m, n, k, schedule]), 2 * copies)
            return graph_us(lambda i: hip.call("nc_matmul_i8_token_acc", [acc, xq, ws[i % copies][0]],
                                               [m, n, k, schedule]), 2 * copies)

        tiles = [t for t in range(16, 32) if (hip.schedule_info(t) or {}).get("kernel") == "mfma"]
        row = {"ours_default": round(ours(0), 2),
               "ours_by_tile": {str(t): round(ours(t), 2) for t in tiles},
               "ours_int32_by_tile": {str(t): round(ours(t, "acc"), 2) for t in tiles}}
        a = torch.from_numpy(rng.integers(-127, 128, (m, k)).astype(np.int8)).cuda()
        bs = [torch.from_numpy(rng.integers(-127, 128, (n, k)).astype(np.int8)).cuda() for _ in range(copies)]
        side = torch.cuda.Stream()
        with torch.cuda.stream(side):
            for b in bs:
                torch._int_mm(a, b.t())
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                for r in range(2 * copies):
                    torch._int_mm(a, bs[r % copies].t())
        graph.replay()
        torch.cuda.synchronize()
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        samples = []
        for _ in range(5):
            start.record()
            graph.replay()
            stop.record()
            torch.cuda.synchronize()
            samples.append(start.elapsed_time(stop) * 1e3 / (2 * copies))
        row["vendor_int_mm"] = round(statistics.median(samples), 2)
        out[name] = row
        log(f"gemms {name}: ours {row['ours_default']} us, torch._int_mm {row['vendor_int_mm']} us")
    return out


# -- config 5: the whole model, greedy decode ----------------------------------------

LM_HEAD_BYTES = 4 * 151936 * 896 + 4 * 896 + 8


def decode_kernel_bytes(label: str, past: int) -> int:
    """Algorithmic bytes of one launch of a decode-step kernel group at the model's widths
    (H 896, MLP 4864, q/k/v rows 1152, 14/2 heads of 64), its token at position ``past``."""
    H, I, W, heads, kv, D = 896, 4864, 1152, 14, 2, 64
    if label == "qkv":           # int8 rows, scales, bias, x, gamma, out
        return W * H + 4 * W + 4 * W + 4 * H + 4 * H + 4 * W
    if label == "attention":     # cached K and V read, the q/k/v row, cos/sin, ctx out, the k/v append
        return 2 * kv * past * D * 4 + 4 * W + 4 * D + 4 * heads * D + 2 * kv * D * 4
    if label == "o":             # int8 rows, scales, ctx, residual read and written
        return H * heads * D + 4 * H + 4 * heads * D + 8 * H
    if label == "gate/up":       # two int8 matrices and scales, x, gamma, h out
        return 2 * I * H + 8 * I + 4 * H + 4 * H + 4 * I
    if label == "down":          # int8 rows, scales, h, residual read and written
        return H * I + 4 * H + 4 * I + 8 * H
    if label == "lm head":       # float32 table, x, the argmax key
        return LM_HEAD_BYTES
    raise KeyError(label)


def decode_kernel_table(model, cache, past: int) -> dict:
    """Each kernel group of one decode step at position ``past``, timed live on the library
    stream: a captured graph of the group's launches (one per layer, each layer's own weights,
    so they stream from HBM as in the step) replayed between HIP events, per launch."""
    from nanocompile_amd import hip
    from nanocompile_amd.kernels import float_bits
    c = model.config
    groups: dict[str, list] = {}
    for label, name, pointers, sizes in model.decode_layer_calls(cache, past):
        groups.setdefault(label, []).append((name, pointers, sizes))
    H, V = c.hidden_size, c.vocab_size
    head = ("nc_lm_head", [None, model.best, model.normed, model.head, model.norm],
            [1, V, H, float_bits(c.rms_norm_eps), 1])
    groups["lm head"] = [head] * 8
    table = {}
    for label, calls in groups.items():
        per_step = 1 if label == "lm head" else len(calls)
        us = graph_us(lambda i, calls=calls: hip.call(*calls[i]), len(calls), rounds=7)
        nbytes = decode_kernel_bytes(label, past)
        table[label] = {"launch_us": round(us, 3), "launches_per_step": per_step,
                        "step_us": round(us * per_step, 2), "bytes_per_launch": nbytes,
                        "gbps": round(nbytes / (us * 1e-6) / 1e9, 1),
                        "frac": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4)}
    return table


def decode_kernels(reps: int = 3, seed: int = 0) -> dict:
    """Each kernel of config 5's decode step at its last position (past 383), launched eagerly over
    the 24 layers' weights ``reps`` times, with no decode loop and no graph: the run rocprofv3's
    counter passes (FETCH_SIZE, WRITE_SIZE) profile for each kernel's HBM traffic. Returns each
    kernel's mean launch time from events around the eager launches."""
    from nanocompile_amd import hip
    from nanocompile_amd.hip import Event
    from nanocompile_amd.kernels import float_bits
    from nanocompile_amd.models.config import QWEN25_05B, random_weights
    from nanocompile_amd.models.qwen2 import Qwen2

    config = QWEN25_05B
    model = Qwen2(config, random_weights(config, seed=seed), max_tokens=PROMPT)
    cache = model.new_cache(PROMPT + NEW_TOKENS)
    past = PROMPT + NEW_TOKENS - 2
    groups: dict[str, list] = {}
    for label, name, pointers, sizes in model.decode_layer_calls(cache, past):
        groups.setdefault(label, []).append((name, pointers, sizes))
    c = config
    groups["lm head"] = [("nc_lm_head", [None, model.best, model.normed, model.head, model.norm],
                          [1, c.vocab_size, c.hidden_size, float_bits(c.rms_norm_eps), 1])]
    out = {}
    for label, calls in groups.items():
        a, b = Event(), Event()
        a.record()
        for _ in range(reps):
            for call in calls:
                hip.call(*call)
        b.record()
        hip.sync()
        out[label] = {"kernel": KERNEL_SYMBOLS[label], "launch_us": round(a.elapsed_ms(b) * 1e3 / (reps * len(calls)), 3),
                      "bytes_per_launch": decode_kernel_bytes(label, past), "launches": reps * len(calls)}
    return out


def cpu_decode(config, weights, prompt, gpu_tokens, seconds: float = 16.0) -> dict:
    """The host C int8 model (oracle/nc_model.c) on this machine's cores: every token checked
    against the GPU's, then a thread sweep of decode steps at the config's positions."""
    from oracle import host
    from oracle.host_model import HostQwen2
    cores = os.cpu_count() or 1
    counts = sorted({1, 2, 4, 8, 16, min(cores, 64)} & set(range(1, min(cores, 64) + 1)))
    t0 = time.perf_counter()
    ref = HostQwen2(config, weights, capacity=PROMPT + NEW_TOKENS)
    log(f"cpu: host model built in {time.perf_counter() - t0:.1f} s")
    host.set_threads(counts[-1])
    t0 = time.perf_counter()
    _, first = ref.forward(prompt)
    prefill_s = time.perf_counter() - t0
    tokens = [first]
    t0 = time.perf_counter()
    for _ in range(NEW_TOKENS - 1):
        tokens.append(ref.forward([tokens[-1]])[1])
    all_cores_full = (NEW_TOKENS - 1) / (time.perf_counter() - t0)
    if tokens != gpu_tokens:
        first_diff = next(i for i, (a, b) in enumerate(zip(tokens, gpu_tokens)) if a != b)
        log(f"cpu: TOKENS DIFFER from the GPU's at position {first_diff}")
    # the sweep: each thread count decodes steps at the config's last positions (past 383 - n
    # .. 382), feeding the same tokens, for about seconds / len(counts) each
    rates = {}
    for t in counts:
        host.set_threads(t)
        n = max(2, min(NEW_TOKENS - 2, int(seconds / len(counts) * (all_cores_full if t == counts[-1]
                                                                          else all_cores_full * t / counts[-1]))))
        ref.length = PROMPT + NEW_TOKENS - 1 - n
        t0 = time.perf_counter()
        for j in range(n):
            ref.forward([tokens[NEW_TOKENS - 1 - n + j]])
        rates[t] = n / (time.perf_counter() - t0)
    best = max(rates, key=rates.get)
    return {"tok_s": rates[best], "threads": best, "all_cores_tok_s": rates[counts[-1]],
            "all_cores": counts[-1], "by_threads": {str(k): round(v, 2) for k, v in rates.items()},
            "full_run_tok_s": all_cores_full, "prefill_s": prefill_s, "cores": cores, "isa": host.isa(),
            "tokens_identical": tokens == gpu_tokens}


REFERENCE_PUBLISHED_TOK_S = {"int8": 21.22, "int8-vnni": 19.77}     # README.md:718-719, i7-12700H, 6 threads


def reference_modes(weights, prompt, seed: int, graph: bool = True) -> dict:
    """Config 5 in the reference's own int8 modes on the hand-written model: ``int8`` (float32
    activations into matmul_i8's 32-chain order) and ``int8-vnni`` (32-wide int8 activation
    blocks into matmul_i8_vnni's order), each decoding the 256 greedy tokens with one graph
    replay a token. Timed over all 255 replays with HIP events; the tokens are compared with the
    reference's own run of this workload (golden G6, tests/golden/g6.json, seed 0) and set beside
    the reference's published CPU figures for these modes."""
    from nanocompile_amd.hip import Event
    from nanocompile_amd.models.config import QWEN25_05B
    from nanocompile_amd.models.qwen2 import Qwen2
    g6 = json.loads((Path(__file__).resolve().parent / "tests" / "golden" / "g6.json").read_text())
    comparable = seed == g6["seed"] and prompt == g6["prompt"]
    replays = NEW_TOKENS - 1
    out = {}
    for mode, tag in (("int8", "int8"), ("int8-vnni", "vnni")):
        t0 = time.perf_counter()
        model = Qwen2(QWEN25_05B, weights, quantization=mode, max_tokens=PROMPT)
        built = time.perf_counter() - t0
        marks = {0: Event(), replays: Event()}
        tokens = model.generate(prompt, NEW_TOKENS, timer=lambda i: marks[i].record() if i in marks else None,
                                graph=graph)
        ms = marks[0].elapsed_ms(marks[replays])
        same = {key: (tokens == g6[key]["tokens"][:NEW_TOKENS]) if comparable else None
                for key in (tag, f"{tag}_ncmath")}
        out[mode] = {"tok_s": round(replays / (ms * 1e-3), 2), "ms_per_step": round(ms / replays, 4),
                     "tokens_identical_to_reference": same[tag],
                     "tokens_identical_to_reference_same_math": same[f"{tag}_ncmath"],
                     "reference_published_cpu_tok_s": REFERENCE_PUBLISHED_TOK_S[mode], "model_build_s": round(built, 1)}
        log(f"reference modes: {mode} {out[mode]['tok_s']} tok/s, tokens identical to the reference's run: "
            f"{same[tag]} (with the C library's exp/sin/cos), {same[f'{tag}_ncmath']} (with this package's)")
        del model
    out["note"] = ("all 255 decode replays after the 128-token prompt, events on the library stream; the reference's "
                   "published figures are its own CPU runs (README.md:718-719), a different machine and real weights; "
                   "int8-vnni's tokens follow the reference's run with the same exp/sin/cos (the mode rounds its "
                   "activations at every projection, so the C library's last-bit differences move its tokens)")
    return out


def qwen2_graph_interface(config, mode: str, last_only: bool = True):
    """What HIPBackend reads of the reference's Qwen2 graph (models/qwen2.py:167-224 after
    quantize.quantize): its name, inputs, outputs, the weights it reads and its int8 primitive.
    The reference's graphs at the tiny model's size are recorded in tests/golden/runner_graphs.json
    (the backend is tested on those); this is the same interface at config 5's size."""
    from types import SimpleNamespace

    from nanocompile_amd.runner import HIPBackend
    weights = HIPBackend(config).expected_weights(mode)
    op = {"int8": "matmul_i8", "int8-vnni": "matmul_i8_vnni"}.get(mode)
    nodes = [SimpleNamespace(op=op, attrs={"block": 32} if mode == "int8-vnni" else {})] if op else []
    return SimpleNamespace(
        name="qwen2_last" if last_only else "qwen2",
        inputs=[SimpleNamespace(attrs={"name": n}) for n in ("token_ids", "past_keys", "past_values")],
        outputs={"logits": None, "keys": None, "values": None},
        weights={name: SimpleNamespace(dtype=dtype, shape=list(shape)) for name, (dtype, shape) in weights.items()},
        nodes=nodes)


def runner_decode(weights, prompt, expected: list[int], activations: str) -> dict:
    """Config 5 through the reference's Runner protocol (models/qwen2.py:229, 316-368): the
    reference's greedy loop restated over ``HIPBackend`` and a host cache kept the reference's way
    (one buffer sized for the sequence, a view of its filled rows handed over each call, the new
    keys and values appended after them). Each call uploads the token, runs the model, and
    downloads the logits row and the new keys and values; argmax on the host. Host wall time of
    the 255 decode calls (every call ends in a wait for its results)."""
    from nanocompile_amd import hip, kernels
    from nanocompile_amd.models.config import QWEN25_05B as c
    from nanocompile_amd.runner import HIPBackend
    graph = qwen2_graph_interface(c, "int8")
    passed = {}
    for name in HIPBackend(c).expected_weights("int8"):
        if name.endswith("@int8"):
            w = name.rsplit("@", 1)[0]
            q, scales = kernels.quantize_int8(weights[w])          # quantize.py:55-70, on the GPU
            passed[name], passed[w + "@scales"] = q.numpy(), scales.numpy()
        elif not name.endswith("@scales"):
            passed[name] = weights[name]
    backend = HIPBackend(c, max_tokens=PROMPT, activations=activations)
    shape = (c.num_hidden_layers, c.num_key_value_heads, PROMPT + NEW_TOKENS, c.head_dim)
    keys, values, length = np.zeros(shape, np.float32), np.zeros(shape, np.float32), 0
    pending, tokens, started = list(prompt), [], None
    before = None
    for i in range(NEW_TOKENS):
        if i == 1:
            started, before = time.perf_counter(), hip.allocations()
        out = backend(graph, {"token_ids": np.asarray(pending, np.int64), "past_keys": keys[:, :, :length],
                              "past_values": values[:, :, :length]}, passed)
        n = out["keys"].shape[2]
        keys[:, :, length:length + n], values[:, :, length:length + n] = out["keys"], out["values"]
        length += n
        tokens.append(int(np.argmax(out["logits"][0])))
        pending = [tokens[-1]]
    seconds = time.perf_counter() - started
    return {"tok_s": round((NEW_TOKENS - 1) / seconds, 2), "ms_per_step": round(seconds * 1e3 / (NEW_TOKENS - 1), 3),
            "activations": activations, "device_allocations_after_first_call": hip.allocations() - before,
            "tokens_identical_to_device_loop": tokens == expected if expected is not None else None}


def decode(steps: int, warmup: int, cpu: bool, seed: int = 0, graph: bool = True, blocks: bool = True) -> dict:
    """Config 5 as stated: 256 greedy tokens after the 128-token prompt, whatever ``steps`` is;
    the last ``steps`` of the 255 replays (ending at past 383, the config's expensive end) are
    the timed region, and the mean over all 255 is reported beside them."""
    from nanocompile_amd.hip import Event
    from nanocompile_amd.models.config import QWEN25_05B
    from nanocompile_amd.models.config import random_weights
    from nanocompile_amd.models.qwen2 import Qwen2

    config = QWEN25_05B
    replays = NEW_TOKENS - 1
    if not 1 <= steps <= replays:
        raise SystemExit(f"--steps {steps}: config 5 has {replays} decode steps after the prompt's token")
    t0 = time.perf_counter()
    weights = random_weights(config, seed=seed)
    prompt = [int(t) for t in np.random.default_rng(seed + 1).integers(0, config.vocab_size, PROMPT)]
    log(f"decode: weights drawn in {time.perf_counter() - t0:.1f} s")
    t0 = time.perf_counter()
    model = Qwen2(config, weights, max_tokens=512)        # 512: config 4's prefill length
    log(f"decode: model uploaded and quantized on the GPU in {time.perf_counter() - t0:.1f} s")

    for _ in range(warmup):
        model.generate(prompt, 16, graph=graph)
    marks = {0: Event(), replays - steps: Event(), replays: Event()}

    def timer(i: int) -> None:
        if i in marks:
            marks[i].record()

    t0 = time.perf_counter()
    tokens = model.generate(prompt, NEW_TOKENS, timer=timer, graph=graph)
    wall = time.perf_counter() - t0
    timed_ms = marks[replays - steps].elapsed_ms(marks[replays])
    all_ms = marks[0].elapsed_ms(marks[replays])
    # the timed replays run at past PROMPT + replays - steps .. PROMPT + replays - 1
    mean_past = PROMPT + replays - (steps + 1) / 2
    result = {"tokens": tokens, "timed_ms": timed_ms, "steps": steps, "wall_s": wall,
              "tok_s": steps / (timed_ms * 1e-3), "all_ms": all_ms, "all_tok_s": replays / (all_ms * 1e-3),
              "step_bytes": 904_503_808 + 24_576 * mean_past}
    cache = model.new_cache(PROMPT + NEW_TOKENS)
    result["kernels"] = decode_kernel_table(model, cache, PROMPT + replays - 1)
    if blocks:
        t0 = time.perf_counter()
        result["blocks"] = block_measurements(model)
        log(f"blocks: configs 2-4 measured in {time.perf_counter() - t0:.1f} s")
        t0 = time.perf_counter()
        result["generated"] = generated_config5(weights)
        log(f"generated: config 5's reference program as HIP, {result['generated']['default']['tok_s']} tok/s "
            f"default, {result['generated']['tuned']['tok_s']} tuned, in {time.perf_counter() - t0:.1f} s")
    if blocks:
        t0 = time.perf_counter()
        result["reference_modes"] = reference_modes(weights, prompt, seed, graph=graph)
        result["runner"] = {"token": runner_decode(weights, prompt, tokens, "token")}
        log(f"runner: config 5 through the reference's Runner protocol, per-token activations: "
            f"{result['runner']['token']['tok_s']} tok/s; reference modes and runner in {time.perf_counter() - t0:.1f} s")
    if cpu:
        result["cpu"] = cpu_decode(config, weights, prompt, tokens)
    return result


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=NEW_TOKENS - 1)
    parser.add_argument("--warmup", type=int, default=1)
    parser.add_argument("--workload", choices=("decode", "gemv", "kernels", "generated", "generated5", "generated4",
                                               "gemms", "modes"),
                        default="decode",
                        help="kernels: each decode-step kernel launched eagerly at past 383 (for counter passes); "
                             "generated / generated5 / generated4: config 2's generated programs / config 5's generated "
                             "decode step, default and tuned, launched eagerly (for kernel traces); gemms: config 4's "
                             "int8 GEMMs, every MFMA tile, against the vendor library's int8 GEMM; modes: config 5 in "
                             "the reference's int8 and int8-vnni modes alone (with --no-graph, launched eagerly)")
    parser.add_argument("--no-cpu", action="store_true")
    parser.add_argument("--no-blocks", action="store_true", help="skip the per-block measurements (configs 2-4)")
    parser.add_argument("--no-graph", action="store_true",
                        help="launch each decode step's kernels directly instead of replaying a HIP graph "
                             "(for profilers that cannot follow graph launches)")
    args = parser.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only: this build has no multi-GPU path (asked for --gpus {args.gpus})",
              file=sys.stderr)
        return 2
    if args.workload == "gemms":
        print(json.dumps({"workload": "config 4's int8 GEMMs at 512 rows against torch._int_mm, graph-replayed",
                          "us": prefill_gemms_vs_library()}), flush=True)
        return 0
    from nanocompile_amd import hip
    from nanocompile_amd.hip import DeviceArray
    hip.init(0)
    info = hip.device_info()
    calibration = CALIBRATION_BYTES
    src, dst = DeviceArray((calibration,), np.uint8), DeviceArray((calibration,), np.uint8)
    hip.load().nc_memcpy_d2d(dst.ptr, src.ptr, calibration)
    hip.sync()
    del src, dst

    if args.workload == "generated4":
        from nanocompile_amd.models.config import QWEN25_05B, random_weights
        print(json.dumps({"workload": "config 4 through the reference's program as HIP: a 512-token prompt's "
                                      "prefill, 24 layers, past 0",
                          **generated_config5(random_weights(QWEN25_05B, seed=0), past=0, seq=512, cache=True,
                                              eager=3, rounds=3, reps=2)}), flush=True)
        return 0
    if args.workload == "generated5":
        from nanocompile_amd.models.config import QWEN25_05B, random_weights
        print(json.dumps({"workload": "config 5's reference program as HIP, one decode step at past 382, eager",
                          **generated_config5(random_weights(QWEN25_05B, seed=0), cache=True, eager=10)}),
              flush=True)
        return 0
    if args.workload == "generated":
        print(json.dumps({"workload": "config 2's generated programs at 512 rows, eager",
                          **generated_kernels()}), flush=True)
        return 0
    if args.workload == "kernels":
        print(json.dumps({"workload": "config 5's decode-step kernels, eager, past 383",
                          "kernels": decode_kernels()}), flush=True)
        return 0
    if args.workload == "modes":
        from nanocompile_amd.models.config import QWEN25_05B, random_weights
        weights = random_weights(QWEN25_05B, seed=0)
        prompt = [int(t) for t in np.random.default_rng(1).integers(0, QWEN25_05B.vocab_size, PROMPT)]
        print(json.dumps({"workload": "config 5 in the reference's own modes, 256 greedy tokens after the "
                                      "128-token prompt" + (", eager" if args.no_graph else ""),
                          **reference_modes(weights, prompt, 0, graph=not args.no_graph)}), flush=True)
        return 0
    g = gpu_gemv(20 if args.workload == "decode" else args.steps, 3)
    log(f"gemv: stacked {g['stacked_gbps']:.0f} GB/s, single {g['single_us']:.2f} us")
    gemv_record = {"stacked_gbps": round(g["stacked_gbps"], 1), "frac": round(g["stacked_gbps"] / HBM_PEAK_GBPS, 4),
                   "stacked_ms": round(g["stacked_ms"], 4), "schedule": g["schedule"],
                   "stacked_gbps_by_schedule": g["by_schedule_gbps"],
                   "single_launch_us": round(g["single_us"], 3), "single_launch_schedule": 0,
                   "single_launch_gbps": round(g["single_gbps"], 1), "copies_per_launch": COPIES,
                   "kernel": f"gemv_i8_token<896, {g['lanes_per_row']}, {g['waves']}, 1, false, true> (stacked)"}
    if args.workload == "gemv":
        cpu = None if args.no_cpu else cpu_gemv()
        record = {
            "metric": "int8 GEMV HBM GB/s (decode projection [1,896]x[4864,896]^T)", "value": round(g["stacked_gbps"], 1),
            "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": 3, "ms_per_step": round(g["stacked_ms"], 4),
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8",
            "data": "synthetic (seeded N(0,0.02) weights, N(0,1) activations)",
            "config": {"workload": "config 1: decode GEMV, per-token int8 x per-row int8", "device": info["arch"]},
            "roofline": {"bound": "hbm", "achieved": round(g["stacked_gbps"], 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                         "frac": round(g["stacked_gbps"] / HBM_PEAK_GBPS, 4),
                         "traffic": measured_traffic(gemv_record["kernel"]),
                         "traffic_source": "profiles/traffic.json (rocprofv3 PMC, calibrated)",
                         "kernel": gemv_record["kernel"], "bytes_per_launch": g["per_launch_bytes"]},
            "cpu_baseline": None if cpu is None else {
                "value": round(cpu["gbps"], 2), "unit": "GB/s", "cores": cpu["threads"], "kind": "port",
                "sample": "240 rotated weight copies", "isa": cpu["isa"], "by_threads": cpu["by_threads"]},
        }
        print(json.dumps(record), flush=True)
        return 0

    global USE_GRAPHS
    USE_GRAPHS = not args.no_graph
    d = decode(args.steps, args.warmup, cpu=not args.no_cpu, graph=not args.no_graph, blocks=not args.no_blocks)
    kernels = d["kernels"]
    # the roofline's kernel is the single kernel with the most time a step; attention's entry
    # point is two kernels (chunks, combine), timed together, so it is reported beside it
    single = [k for k in kernels if " + " not in KERNEL_SYMBOLS[k]]
    dominant = max(single, key=lambda k: kernels[k]["step_us"])
    top = kernels[dominant]
    log(f"decode: {d['tok_s']:.1f} tok/s on the GPU (last {args.steps} replays), {d['all_tok_s']:.1f} over all "
        f"{NEW_TOKENS - 1}; time-dominant kernel {dominant}: {top['step_us']:.1f} us a step")
    cpu = d.get("cpu")
    cpu_g = None if args.no_cpu else cpu_gemv(seconds=8.0)
    cpu_b = None if args.no_cpu else cpu_blocks()
    read = None if args.no_cpu else host_read_bandwidth()
    step_gbps = d["step_bytes"] * d["tok_s"] / 1e9
    record = {
        "metric": "decode tok/s, Qwen2-0.5B-shape int8 on 1 MI355X",
        "value": round(d["tok_s"], 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(d["timed_ms"] / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (random-init weights N(0,0.02), uniform-random 128-token prompt)",
        "config": {"workload": "config 5: Qwen2.5-0.5B-shaped, int8 projections with per-token int8 activations, "
                               "fp32 tied LM head; 128-token prompt then 256 greedy tokens (past to 384); the "
                               "timed steps are the last `steps` decode replays, ending at past 383",
                   "prompt_tokens": PROMPT, "new_tokens": NEW_TOKENS, "device": info["arch"],
                   "compute_units": info["compute_units"],
                   "tokens_identical_to_host_c": None if cpu is None else cpu["tokens_identical"],
                   "tokens_checked": NEW_TOKENS,
                   "all_replays": {"replays": NEW_TOKENS - 1, "ms": round(d["all_ms"], 3),
                                   "tok_s": round(d["all_tok_s"], 2)},
                   "kernels_per_step": kernels,
                   "gemv": gemv_record,
                   "blocks": d.get("blocks"),
                   "generated": d.get("generated"),
                   "reference_modes": d.get("reference_modes"),
                   "runner": d.get("runner")},
        "roofline": {"bound": "hbm", "achieved": top["gbps"], "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": top["frac"], "traffic": measured_traffic(KERNEL_SYMBOLS[dominant]),
                     "traffic_source": "profiles/traffic.json (rocprofv3 PMC, calibrated); null when no pass "
                                       "exists for this kernel (profiles/decode_step_config5.md)",
                     "kernel": f"{KERNEL_SYMBOLS[dominant]} ({dominant}: the decode step's time-dominant kernel, "
                               f"{top['launches_per_step']} launches, {top['step_us']} us a step)",
                     "bytes_per_launch": top["bytes_per_launch"], "launch_us": top["launch_us"],
                     "step": {"bytes": int(d["step_bytes"]), "gbps": round(step_gbps, 1),
                              "frac": round(step_gbps / HBM_PEAK_GBPS, 4)},
                     "lm_head": kernels["lm head"],
                     "attention": dict(kernels["attention"], kernels=KERNEL_SYMBOLS["attention"])},
        "cpu_baseline": None if cpu is None else {
            "value": round(cpu["tok_s"], 2), "unit": "tok/s", "cores": cpu["threads"], "kind": "port",
            "sample": f"decode steps at the config's last positions on the host C int8 model (oracle/nc_model.c, "
                      f"the build's own C: the reference has no per-token int8 mode), {cpu['isa']}; threads swept "
                      f"{list(cpu['by_threads'])}, best {cpu['threads']}",
            "by_threads": cpu["by_threads"], "all_cores": cpu["all_cores"],
            "all_cores_tok_s": round(cpu["all_cores_tok_s"], 2), "host_cores": cpu["cores"],
            "full_run_tok_s": round(cpu["full_run_tok_s"], 2), "prefill_s": round(cpu["prefill_s"], 3),
            "gemv": None if cpu_g is None else {
                "value": round(cpu_g["gbps"], 2), "unit": "GB/s", "threads": cpu_g["threads"],
                "by_threads": cpu_g["by_threads"], "isa": cpu_g["isa"],
                "all_cores_gbps": cpu_g["by_threads"][str(max(map(int, cpu_g["by_threads"])))],
                "sample": "config 1's GEMV over 240 rotated weight copies (1 GB, past the host's LLC)"},
            "blocks": cpu_b,
            "host_read_gbps": None if read is None else read["gbps"],
            "host_read": read,
            "fraction_of_host_read": None if read is None else host_fractions(read["gbps"], cpu, cpu_g, cpu_b, d)},
    }
    print(json.dumps(record), flush=True)
    return 0


def host_read_bandwidth() -> dict:
    """The host's measured read bandwidth (oracle/nc_host.c nc_host_read_gbps: every core summing
    its share of a 1 GiB buffer, the reference's bench/probe.c:47-72 idea), the denominator of
    each CPU figure's fraction."""
    from oracle import host
    cores = os.cpu_count() or 1
    threads = min(cores, 64)
    host.set_threads(threads)
    host.read_gbps(1 << 30, 1)                     # pages touched, threads up
    gbps = max(host.read_gbps(1 << 30, 3) for _ in range(3))
    log(f"cpu: host read bandwidth {gbps:.1f} GB/s on {threads} threads")
    return {"gbps": round(gbps, 2), "threads": threads, "buffer_bytes": 1 << 30,
            "method": "int64 sums over 256 chunks of a 1 GiB buffer on the host pool, best of 3 x 3 passes"}


def host_fractions(read: float, cpu, cpu_g, cpu_b, d) -> dict:
    """Each host figure's bytes per second over the host's read bandwidth."""
    out = {}
    if cpu is not None:
        out["decode"] = round(d["step_bytes"] * cpu["tok_s"] / 1e9 / read, 4)
    if cpu_g is not None:
        out["gemv"] = round(cpu_g["gbps"] / read, 4)
    if cpu_b is not None:
        out["rms_norm_quant_512"] = round(cpu_b["rms_norm_quant_512"]["gbps"] / read, 4)
        out["block_decode"] = round(cpu_b["block_decode"]["gbps"] / read, 4)
    return out


if __name__ == "__main__":
    raise SystemExit(main())
