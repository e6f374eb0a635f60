"""Every point of the generated kernels' schedule space on the GPU, and the tuner that chooses.

For each program of ``candidate_programs`` (each zoo graph as fused, and
config 2's graph unfused), every candidate schedule of every kernel (thread
counts, LDS staging, workgroup items, vector widths, unroll: gpu_schedule.space)
is generated into one library (autotune.CandidateLibrary) and the program
runs the recorded cases with each kernel at each of its candidates in turn:
its outputs must be the reference C's, bit for bit except outputs computed
through exp, sin or cos (the reference's own tolerance), and an out-of-range
gather must still raise KernelError. A staged window too large for LDS at run
time takes the unstaged kernel, bitwise the same. The tuner checks every
candidate against the default on the same arguments before timing it, and
its choice, run from the same library, gives the reference's outputs; a
second tuner with the same cache measures nothing.
"""

from __future__ import annotations

import numpy as np
import pytest

from tests import programs as P
from tests.conftest import bits
from tests.test_codegen_gpu import check

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name,variant", P.candidate_programs())
def test_every_candidate_of_every_kernel_is_the_references_c(gpu, name, variant):
    from nanocompile_amd import autotune
    from nanocompile_amd.compiled import CompiledProgram
    from nanocompile_amd.hip import KernelError
    library = autotune.CandidateLibrary(P.zoo(name, variant))
    cases, weights = P.zoo_cases(name)
    most = max(len(c) for c in library.candidates)
    print(f"candidates {name} {variant}: {[len(c) for c in library.candidates]}", flush=True)
    for k in range(most):
        chosen = [k % len(c) for c in library.candidates]
        compiled = CompiledProgram(library.program, autotune.Chosen(library, chosen))
        for inputs, want, error in cases:
            if error is not None:
                with pytest.raises(KernelError, match="outside"):
                    compiled(inputs, weights)
                continue
            try:
                check(name, compiled(inputs, weights), want)
            except AssertionError as e:
                where = [library.candidates[i][c].launch.describe() for i, c in enumerate(chosen)]
                raise AssertionError(f"{e}\nschedules: {where}") from None


def test_a_window_too_large_for_lds_takes_the_unstaged_kernel(gpu):
    """softmax_mask's row kernel stages its row of past + seq floats: at past 20000 (80 KB) the
    launcher takes the unstaged kernel, at past 1000 the staged one; both are the default's bits."""
    from nanocompile_amd import autotune, gpu_schedule
    from nanocompile_amd.compiled import CompiledProgram
    library = autotune.CandidateLibrary(P.zoo("softmax_mask"))
    row = next(i for i, k in enumerate(library.program.kernels) if gpu_schedule.kernel_class(k) == "row")
    staged = [c for c, cand in enumerate(library.candidates[row]) if cand.launch.stage]
    assert staged
    default = CompiledProgram(library.program, autotune.Chosen(library, [0] * len(library.candidates)))
    rng = np.random.default_rng(5)
    for past in (1000, 20000):
        seq = 3
        inputs = {"s": rng.standard_normal((2, seq, past + seq)).astype(np.float32),
                  "anchor": np.zeros(past, np.float32)}
        want = default(inputs, {})
        for c in staged[:4]:
            chosen = [0] * len(library.candidates)
            chosen[row] = c
            got = CompiledProgram(library.program, autotune.Chosen(library, chosen))(inputs, {})
            for key in want:
                assert np.array_equal(bits(got[key]), bits(want[key])), (past, c, key)


@pytest.mark.parametrize("name,variant", [("rms_norm_quant", "program"), ("rms_norm_quant", "unfused"),
                                          ("softmax_mask", "program"), ("reductions", "program"),
                                          ("gather", "program")])
def test_tuner_checks_every_candidate_and_its_choice_is_the_references_c(gpu, tmp_path, name, variant):
    from nanocompile_amd import autotune
    from nanocompile_amd.compiled import CompiledProgram
    print(f"tune {name} {variant}", flush=True)
    cache = tmp_path / "tuning.json"
    tuner = autotune.Autotuner(rounds=2, reps=4, cache=cache)
    compiled = CompiledProgram(P.zoo(name, variant), schedule=tuner)
    tuned = [r for r in tuner.records if not r.cached]
    assert tuned and all(r.config is not None and r.winner_cost and r.default_cost for r in tuned)
    cases, weights = P.zoo_cases(name)
    for inputs, want, error in cases:
        if error is None:
            check(name, compiled(inputs, weights), want)
    again = autotune.Autotuner(cache=cache)
    CompiledProgram(P.zoo(name, variant), schedule=again)
    assert again.records and all(r.cached for r in again.records)
    assert [r.config for r in again.records] == [r.config for r in tuned]


def test_tuned_tiny_qwen2_greedy_tokens_and_logits_are_golden(gpu, tmp_path):
    """The tiny Qwen2 (int8 mode) with every generated kernel tuned over its schedule space on the
    reference's decode and prefill workloads: golden G5's greedy tokens, and its logits to the
    same tolerance as the default schedules."""
    from nanocompile_amd import autotune
    from nanocompile_amd.compiled import CompiledProgram
    tuner = autotune.Autotuner(rounds=2, reps=4, cache=tmp_path / "tuning.json")
    compiled = {which: CompiledProgram(P.qwen2(tag, which), schedule=tuner) for tag, which in P.candidate_models()}
    assert tuner.records and all(r.config is not None for r in tuner.records)
    print(f"tuned {len(tuner.records)} kernels, {sum(r.winner != 0 for r in tuner.records)} off their defaults",
          flush=True)
    weights = P.qwen2_weights("int8")
    driver = P.Driver(lambda which, inputs: compiled[which](inputs, weights))
    golden = np.load(P.GOLDEN / "golden.npz")
    for i, prompt in enumerate(P.PROMPTS):
        assert driver.greedy(prompt, 8) == list(golden[f"g5_int8_tokens_{i}"]), prompt
    ids = P.PROMPTS[3]
    want = golden["g5_int8_logits"]
    np.testing.assert_allclose(driver.forward(ids), want, rtol=0, atol=1e-5 * np.abs(want).max())


def test_an_item_storing_its_lane_held_accumulators_directly(gpu):
    """``y[i, e] = acc[e]`` with acc held one element a lane: each stored value is a shuffle from
    lane e that every lane of the item evaluates, lane 0 alone storing. Bitwise the direct
    chain of fused multiply-adds, and the unscheduled (default) kernel's output."""
    from nanocompile_amd.compiled import CompiledProgram
    program = P.lane_store_program()
    x = np.random.default_rng(3).standard_normal((3, 32)).astype(np.float32)
    want = P.lane_store_expected(x)
    print("lane_store: lanes and default schedules", flush=True)
    for schedule in (P.lane_store_lanes, "default"):
        got = CompiledProgram(program, schedule)({"x": x}, {})["y"]
        assert np.array_equal(bits(got), bits(want)), schedule
