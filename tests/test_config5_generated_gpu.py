"""Config 5 through the drop-in path: the reference's own compiled program, generated as HIP.

The fixture holds the reference's compilation of config 5's model
(Qwen2.5-0.5B-shaped, 24 layers, vocabulary 151,936, int8 projections with
BASELINE's seeded N(0, 0.02) weights) as a loop-IR program, a seeded
16-token prompt, the four tokens the reference's greedy loop (its compiled
C, models/qwen2.py:348-368) produced from it, and the reference's logits of
the prompt's last position and of the first decode step at every 97th
vocabulary entry. Here that program runs as codegen_hip generated it, on the
GPU, through the reference's forward and greedy loop (tests/programs.Driver):
the same greedy tokens, the same argmax and maximum logit, and the sampled
logits to the tolerance the tiny model's generated logits are held to (the
reference's exp, sin and cos against this package's, within an ulp, through
24 layers).
"""

from __future__ import annotations

import numpy as np
import pytest

from tests import programs as P

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def config5(gpu):
    from nanocompile_amd.compiled import CompiledProgram
    from nanocompile_amd.models.config import QWEN25_05B
    program, record = P.config5()
    print("config 5 generated: building weights", flush=True)
    weights = P.config5_weights(record["weight_names"], record["seed"])
    compiled = CompiledProgram(program)
    driver = P.Driver(lambda which, inputs: compiled(inputs, weights), config=QWEN25_05B)
    driver.program, driver.weights = program, weights
    return driver, record


def _close(got: np.ndarray, record: dict, which: str) -> None:
    want = record[f"logits_{which}"]
    sampled = got[::record["stride"]]
    assert sampled.shape == want.shape
    np.testing.assert_allclose(sampled, want, rtol=0, atol=1e-5 * np.abs(want).max(), err_msg=which)
    assert int(np.argmax(got)) == record[f"argmax_{which}"], which
    assert float(np.max(got)) == pytest.approx(float.fromhex(record[f"max_{which}"]), rel=1e-5, abs=1e-6)


def test_config5_prompt_and_decode_logits_are_the_references(config5):
    driver, record = config5
    print("config 5 generated: prompt", flush=True)
    cache = list(driver.empty())
    first = driver.forward(record["prompt"], cache, last_only=True)[0]
    _close(first, record, "prompt")
    step = driver.forward([int(np.argmax(first))], cache, last_only=True)[0]
    _close(step, record, "step")


def test_config5_greedy_tokens_are_the_references(config5):
    driver, record = config5
    print("config 5 generated: greedy", flush=True)
    assert driver.greedy(record["prompt"], len(record["tokens"])) == record["tokens"]


@pytest.mark.parametrize("unroll", [0, 32])
def test_config5_with_its_int8_matmuls_across_lanes_is_the_references(config5, unroll):
    """The same program with every int8 projection's 32 accumulator chains one a lane
    (gpu_schedule lanes), their k loops as written or unrolled 32 steps (152 steps at
    K = 4864, so a remainder): the reference's tokens and logits."""
    from nanocompile_amd import autotune
    from nanocompile_amd.compiled import CompiledProgram
    from nanocompile_amd.models.config import QWEN25_05B
    driver, record = config5
    library = autotune.CandidateLibrary(driver.program)
    chosen = [next((c for c, cand in enumerate(cands) if cand.config.get("lanes") and cand.config["threads"] == 256
                    and cand.config.get("unroll", 0) == unroll), 0) for cands in library.candidates]
    assert sum(1 for c in chosen if c) >= 7
    compiled = CompiledProgram(driver.program, autotune.Chosen(library, chosen))
    lanes = P.Driver(lambda which, inputs: compiled(inputs, driver.weights), config=QWEN25_05B)
    print(f"config 5 generated, matmuls across lanes, unroll {unroll}", flush=True)
    cache = list(lanes.empty())
    first = lanes.forward(record["prompt"], cache, last_only=True)[0]
    _close(first, record, "prompt")
    _close(lanes.forward([int(np.argmax(first))], cache, last_only=True)[0], record, "step")
    assert lanes.greedy(record["prompt"], len(record["tokens"])) == record["tokens"]
