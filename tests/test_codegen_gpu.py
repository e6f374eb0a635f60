"""Generated HIP (codegen_hip.py) against the reference's own compiled C, on the GPU.

Each recorded program (tests/golden/programs.json.gz: what the reference's
compiler made of a zoo of graphs and of the tiny golden Qwen2) is lowered
with its GPU schedules, built, and run through CompiledProgram on the
recorded inputs. Its outputs must be the reference C's bit for bit, except
outputs computed through exp, sin or cos, which are held to the reference's
own tolerance for those functions (rtol 2e-6, atol 1e-6). The fused,
unfused and CPU-scheduled forms of each zoo graph all run; the three tiny
Qwen2 modes run the reference's greedy loop over the recorded graphs and
must give golden G5's tokens and logits. Out-of-range gather ids raise the
reference's KernelError.
"""

from __future__ import annotations

import numpy as np
import pytest

from tests import programs as P
from tests.conftest import bits

pytestmark = pytest.mark.gpu


def check(name: str, got: dict, want: dict) -> None:
    assert got.keys() == want.keys()
    for key in want:
        g, w = got[key], want[key]
        assert g.dtype == w.dtype and g.shape == w.shape, (key, g.dtype, g.shape, w.dtype, w.shape)
        if key in P.approx(name):
            np.testing.assert_allclose(g, w, rtol=P.RTOL, atol=P.ATOL, err_msg=f"{name}.{key}")
        elif g.dtype == np.float32:
            assert np.array_equal(bits(g), bits(w)), f"{name}.{key}: not bitwise the reference's C"
        else:
            assert np.array_equal(g.view(np.uint8), w.view(np.uint8)), f"{name}.{key}"


@pytest.mark.parametrize("variant", ["program", "unfused", "scheduled"])
@pytest.mark.parametrize("name", P.zoo_names())
def test_zoo_graph_is_the_references_c(gpu, name, variant):
    from nanocompile_amd.compiled import CompiledProgram
    from nanocompile_amd.hip import KernelError
    print(f"codegen {name} {variant}", flush=True)
    compiled = CompiledProgram(P.zoo(name, variant))
    cases, weights = P.zoo_cases(name)
    for inputs, want, error in cases:
        if error is not None:
            with pytest.raises(KernelError, match="outside"):
                compiled(inputs, weights)
            continue
        check(name, compiled(inputs, weights), want)


@pytest.fixture(scope="module", params=["f32", "int8", "vnni"])
def tiny(request, gpu):
    from nanocompile_amd.compiled import CompiledProgram
    tag = request.param
    print(f"codegen qwen2 {tag}", flush=True)
    compiled = {which: CompiledProgram(P.qwen2(tag, which)) for which in ("full", "last")}
    weights = P.qwen2_weights(tag)
    return tag, P.Driver(lambda which, inputs: compiled[which](inputs, weights)), compiled, weights


def test_tiny_qwen2_greedy_tokens_are_golden(tiny):
    import numpy as np
    tag, driver, _, _ = tiny
    golden = np.load(P.GOLDEN / "golden.npz")
    for i, prompt in enumerate(P.PROMPTS):
        assert driver.greedy(prompt, 8) == list(golden[f"g5_{tag}_tokens_{i}"]), (tag, prompt)


def test_tiny_qwen2_logits_are_golden(tiny):
    tag, driver, _, _ = tiny
    golden = np.load(P.GOLDEN / "golden.npz")
    ids = P.PROMPTS[3]
    logits = driver.forward(ids)
    want = golden[f"g5_{tag}_logits"]
    # bitwise but for the rare exp/sin/cos ulp (softmax, RoPE, SiLU), then the graph's own arithmetic
    np.testing.assert_allclose(logits, want, rtol=0, atol=1e-5 * np.abs(want).max())
    cache = list(driver.empty())
    driver.forward(ids[:6], cache)
    step = driver.forward(ids[6:7], cache, last_only=True)
    want = golden[f"g5_{tag}_decode_logits"]
    np.testing.assert_allclose(step, want, rtol=0, atol=1e-5 * np.abs(want).max())


def test_token_out_of_range_is_the_references_kernel_error(tiny):
    from nanocompile_amd.hip import KernelError
    _, driver, _, _ = tiny
    with pytest.raises(KernelError, match="gather index 256 is outside 0..255"):
        driver.forward([1, 256])
    driver.forward([1, 2])                          # and the program still runs


def test_memory_plan_reuses_the_arena(tiny):
    """The temporaries share space (a layer's buffers reuse the previous layer's), and the one
    arena holds weights, inputs, outputs and the plan."""
    _, driver, compiled, _ = tiny
    driver.forward(P.PROMPTS[3])
    plan = compiled["full"].last_plan
    assert plan.region_bytes < plan.unshared_bytes
    assert compiled["full"]._arena.nbytes >= compiled["full"]._region + plan.region_bytes


def test_compiled_graph_and_backend_run_any_program_as_generated_code(gpu):
    """The reference's CompiledGraph/CBackend interface (runtime.py:167-337): a program given
    directly, and a graph that is not a Qwen2 forward lowered by a supplied compilation."""
    from types import SimpleNamespace

    from nanocompile_amd.models.config import TINY
    from nanocompile_amd.runner import HIPBackend, HIPCompiledGraph
    cases, weights = P.zoo_cases("rms_norm")
    inputs, want, _ = cases[1]
    compiled = HIPCompiledGraph(program=P.zoo("rms_norm"))
    assert compiled.path == "codegen"
    profile = {}
    check("rms_norm", compiled(inputs, weights, profile=profile), want)
    assert set(profile) == {"row"} and profile["row"] > 0
    graph = SimpleNamespace(name="rms_norm", nodes=[])                  # stands in for the reference's Graph
    lowered = []

    def lower(g, fuse):
        lowered.append((g, fuse))
        return P.zoo("rms_norm", "program" if fuse else "unfused")

    for config in (None, TINY):
        backend = HIPBackend(config, lower=lower)
        check("rms_norm", backend(graph, inputs, weights), want)
        check("rms_norm", backend(graph, inputs, weights), want)        # compiled once per graph
    assert lowered == [(graph, True), (graph, True)]
    unfused = HIPBackend(None, fuse=False, lower=lower)
    check("rms_norm", unfused(graph, inputs, weights), want)
    assert lowered[-1] == (graph, False)
