"""Benchmark of the int8 hot path on one MI355X, with its roofline and the host baseline.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload gemv|decode]

Prints ONE JSON line. The ``gemv`` workload is BASELINE config 1: the decode
projection [1, 896] x [4864, 896]^T, per-row int8 weights, per-token int8
activations, int32 accumulation, fp32 epilogue. Weights are rotated through
128 device copies (560 MB, past the 256 MB Infinity Cache) so reads come from
HBM. A step is one launch of the stacked kernel over all 128 copies (one
decode GEMV per copy); the single-launch rate at the exact shape is reported
beside it.

Roofline numerator: the algorithmic bytes of one GEMV,
N*K + 4N + M*K + 4M + 4MN = 4,397,956 B (int8 weights, f32 scales, int8
activations, f32 token scale, f32 output), times the GEMVs per launch.

The CPU baseline is the host C int8 path (oracle/nc_host.c) on this machine's
cores over the same shapes, its weights rotated through more than twice the
host's last-level cache.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

import numpy as np

HBM_PEAK_GBPS = 8000.0
N, K, M = 4864, 896, 1
COPIES = 128


def gemv_bytes(m: int, n: int, k: int) -> int:
    return n * k + 4 * n + m * k + 4 * m + 4 * m * n


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


# -- the GPU leg ---------------------------------------------------------------


def gpu_gemv(steps: int, warmup: int, seed: int = 0) -> dict:
    from nanocompile_amd import hip, kernels
    from nanocompile_amd.hip import DeviceArray, Event

    hip.init(0)
    info = hip.device_info()
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    x = rng.standard_normal((M, K)).astype(np.float32)
    q1, s1 = kernels.quantize_int8(w)
    xq1, xs1 = kernels.quantize_token(x)

    # 128 copies of the weights at distinct addresses, and of the activations
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

    # parity of what is timed: every copy's output equals the single GEMV's
    single = kernels.matmul_i8_token(xq1, xs1, q1, s1).numpy()
    kernels.matmul_i8_token_stacked(xq, xs, q, ws, out=y)
    stacked = y.numpy()
    if not all(np.array_equal(stacked[c], single) for c in range(COPIES)):
        raise RuntimeError("stacked GEMV differs from the single GEMV")

    # single launches at the exact shape, each bracketed by events
    views = [(xq.view((M, K), offset_bytes=c * M * K), xs.view((M,), offset_bytes=c * M * 4),
              q.view((N, K), offset_bytes=c * N * K), ws.view((N,), offset_bytes=c * N * 4)) for c in range(COPIES)]
    out1 = DeviceArray((M, N), np.float32)
    args_single = [[out1, v[0], v[1], v[2], v[3], None, None] for v in views]
    for a in args_single[:8]:
        hip.call("nc_matmul_i8_token", a, [M, N, K, 0])
    hip.sync()
    starts = [Event() for _ in range(COPIES)]
    stops = [Event() for _ in range(COPIES)]
    for c in range(COPIES):
        starts[c].record()
        hip.call("nc_matmul_i8_token", args_single[c], [M, N, K, 0])
        stops[c].record()
    hip.sync()
    single_us = statistics.median(starts[c].elapsed_ms(stops[c]) * 1e3 for c in range(COPIES))

    # the stacked launch: warmup, then exactly `steps`, each bracketed by events
    stacked_args = [y, xq, xs, q, ws]
    for _ in range(warmup):
        hip.call("nc_matmul_i8_token_stacked", stacked_args, [COPIES, M, N, K, 0])
    hip.sync()
    ev = [(Event(), Event()) for _ in range(steps)]
    t0 = time.perf_counter()
    for a, b in ev:
        a.record()
        hip.call("nc_matmul_i8_token_stacked", stacked_args, [COPIES, M, N, K, 0])
        b.record()
    hip.sync()
    wall = time.perf_counter() - t0
    launch_ms = [a.elapsed_ms(b) for a, b in ev]
    mean_ms = statistics.fmean(launch_ms)
    per_launch_bytes = gemv_bytes(M, N, K) * COPIES
    return {
        "info": info,
        "stacked_ms": mean_ms,
        "stacked_ms_median": statistics.median(launch_ms),
        "stacked_gbps": per_launch_bytes / (mean_ms * 1e-3) / 1e9,
        "single_us": single_us,
        "single_gbps": gemv_bytes(M, N, K) / (single_us * 1e-6) / 1e9,
        "wall_s": wall,
        "per_launch_bytes": per_launch_bytes,
    }


# -- the CPU leg (the oracle's host C path, timed as the baseline) --------------


def cpu_gemv(seconds: float = 12.0, seed: int = 0) -> dict:
    from oracle import build, host

    if not build.LIBRARY.exists():
        build.build()
    rng = np.random.default_rng(seed)
    cores = os.cpu_count() or 1
    copies = 240                                   # 1.05 GB: past twice any host LLC in sight
    q = rng.integers(-127, 128, (copies, N, K), dtype=np.int8)
    ws = (rng.random((copies, N)) * 1e-3).astype(np.float32)
    xq = rng.integers(-127, 128, (M, K), dtype=np.int8)
    xs = np.ones(M, np.float32)
    counts = sorted({1, 2, 4, 8, 16, 32, 64, min(cores, 128)} & set(range(1, min(cores, 128) + 1)))
    per = seconds / max(1, len(counts))
    results = {}
    for t in counts:
        host.set_threads(t)
        s1 = host.time_matmul_i8_token(xq, xs, q, ws, 1)         # one pass: calibrate
        reps = max(1, int(per / max(s1, 1e-6)))
        s = host.time_matmul_i8_token(xq, xs, q, ws, reps)
        results[t] = gemv_bytes(M, N, K) * copies * reps / s / 1e9
    best = max(results, key=results.get)
    return {"gbps_by_threads": {str(k): round(v, 2) for k, v in results.items()}, "best_threads": best,
            "best_gbps": results[best], "all_threads": counts[-1], "all_gbps": results[counts[-1]],
            "isa": host.isa(), "cores": cores, "sample": f"{copies} rotated weight copies, thread sweep {counts}"}


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=20)
    parser.add_argument("--warmup", type=int, default=3)
    parser.add_argument("--workload", choices=("gemv",), default="gemv")
    parser.add_argument("--cpu-seconds", type=float, default=12.0)
    parser.add_argument("--no-cpu", action="store_true")
    args = parser.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only: this build has no multi-GPU path (asked for --gpus {args.gpus})",
              file=sys.stderr)
        return 2

    log(f"gemv: {COPIES} copies of [{N},{K}] int8, {args.warmup} warmup + {args.steps} steps")
    g = gpu_gemv(args.steps, args.warmup)
    log(f"gpu: stacked {g['stacked_gbps']:.0f} GB/s ({g['stacked_ms']:.3f} ms), "
        f"single {g['single_us']:.2f} us = {g['single_gbps']:.0f} GB/s")
    cpu = None
    if not args.no_cpu:
        cpu = cpu_gemv(args.cpu_seconds)
        log(f"cpu: {cpu['best_gbps']:.1f} GB/s at {cpu['best_threads']} threads ({cpu['isa']})")
    record = {
        "metric": "int8 GEMV HBM GB/s (decode projection, Qwen2-0.5B gate/up shape)",
        "value": round(g["stacked_gbps"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(g["stacked_ms"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded N(0,0.02) weights, N(0,1) activations)",
        "config": {"workload": "config 1: decode GEMV [1,896] x [4864,896]^T, per-token int8 x per-row int8",
                   "copies_per_launch": COPIES, "single_launch_us": round(g["single_us"], 3),
                   "single_launch_gbps": round(g["single_gbps"], 1), "device": g["info"]["arch"],
                   "compute_units": g["info"]["compute_units"]},
        "roofline": {"bound": "hbm", "achieved": round(g["stacked_gbps"], 1), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(g["stacked_gbps"] / HBM_PEAK_GBPS, 4), "traffic": None,
                     "kernel": "gemv_i8_token<896,8,1,1,false,true> (stacked)",
                     "bytes_per_launch": g["per_launch_bytes"]},
        "cpu_baseline": None if cpu is None else {
            "value": round(cpu["best_gbps"], 2), "unit": "GB/s", "cores": cpu["best_threads"], "kind": "port",
            "sample": cpu["sample"], "isa": cpu["isa"], "host_cores": cpu["cores"],
            "all_threads_gbps": round(cpu["all_gbps"], 2), "by_threads": cpu["gbps_by_threads"]},
    }
    print(json.dumps(record), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
