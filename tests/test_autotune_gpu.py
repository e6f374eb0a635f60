"""The autotuner on the GPU: it measures, checks bits, caches, and the model runs on its choices."""

from __future__ import annotations

import numpy as np
import pytest

from nanocompile_amd import autotune
from tests.conftest import bits

pytestmark = pytest.mark.gpu


def test_tune_checks_measures_and_caches(gpu, tmp_path):
    from nanocompile_amd import autotune
    print("autotune matmul_i8_token m=64 n=256 k=256", flush=True)
    cache = tmp_path / "tuning.json"
    tuner = autotune.Autotuner(rounds=3, reps=4, cache=cache, stream_bytes=4 << 20)
    record = tuner.tune("matmul_i8_token", 64, 256, 256)
    space = [c["schedule"] for c in autotune.legal_space("matmul_i8_token", 64, 256, 256)]
    assert record.winner in space and not record.cached
    assert record.evaluations[0].schedules == space
    assert all(c > 0 for c in record.evaluations[0].costs)
    again = autotune.Autotuner(cache=cache).tune("matmul_i8_token", 64, 256, 256)
    assert again.cached and again.winner == record.winner
    swiglu = tuner.tune("matmul_i8_token_swiglu", 32, 128, 128)
    assert swiglu.winner in [c["schedule"] for c in autotune.legal_space("matmul_i8_token_swiglu", 32, 128, 128)]


def test_model_on_tuned_schedules_is_bitwise_the_default(gpu, tmp_path):
    from nanocompile_amd import autotune
    from nanocompile_amd.models.config import TINY, TINY_STD, random_weights
    from nanocompile_amd.models.qwen2 import Qwen2
    print("autotuned tiny model", flush=True)
    weights = random_weights(TINY, seed=3, std=TINY_STD)
    ids = np.random.default_rng(4).integers(0, TINY.vocab_size, 40)
    default = Qwen2(TINY, weights, max_tokens=64)
    tuner = autotune.Autotuner(rounds=3, reps=4, cache=tmp_path / "t.json", stream_bytes=1 << 20)
    tuned = Qwen2(TINY, weights, max_tokens=64, schedule=tuner)
    a = default.forward(ids, default.new_cache(64))
    b = tuned.forward(ids, tuned.new_cache(64))
    assert np.array_equal(bits(a), bits(b))
    assert {r.op for r in tuner.records} == {"matmul_i8_token", "matmul_i8_token_swiglu", "attention_prefill",
                                            "qkv_rope"}
    assert tuned.generate(list(ids[:8]), 6) == default.generate(list(ids[:8]), 6)


@pytest.mark.parametrize("kind,n,k", [(0, 1152, 896), (1, 896, 896), (2, 4864, 896), (1, 896, 4864)])
def test_every_decode_projection_schedule_is_the_default_bitwise(gpu, kind, n, k):
    """nc_decode_projection's launch shapes (nc_decode_schedule_info) all compute schedule 0's bits,
    inside guard regions, on the model's four one-token projections."""
    problem = autotune.DecodeProblem(kind, n, k, seed=kind + n, stream_bytes=1 << 20)
    space = problem.space()
    assert len(space) >= 4
    reference = problem.output(0)
    for candidate in space[1:]:
        print(f"decode kind {kind} ({n}, {k}) schedule {candidate}", flush=True)
        assert np.array_equal(problem.output(candidate["schedule"]), reference), candidate


@pytest.mark.parametrize("m", [7, 130, 512])
def test_every_prefill_attention_schedule_is_the_default_bitwise(gpu, m):
    problem = autotune.AttentionProblem(m, 14, 2, 64, seed=m)
    reference = problem.output(0)
    for candidate in problem.space()[1:]:
        print(f"attention m={m} schedule {candidate}", flush=True)
        assert np.array_equal(problem.output(candidate["schedule"]), reference), candidate


@pytest.mark.parametrize("m", [16, 130, 512])
def test_every_qkv_rope_schedule_is_the_default_bitwise(gpu, m):
    """The fused qkv + RoPE + cache-append GEMM: every tile one head wide leaves qkv and both
    caches as the library's choice does."""
    problem = autotune.RopeProblem(m, 1152, 896, 14, 2, 64, seed=m, stream_bytes=4 << 20)
    space = problem.space()
    assert [c["schedule"] for c in space] == [0, 16, 17, 20, 21, 24]
    reference = problem.output(0)
    for candidate in space[1:]:
        print(f"qkv rope m={m} schedule {candidate['schedule']}", flush=True)
        assert np.array_equal(problem.output(candidate["schedule"]), reference), candidate


def test_tuner_chooses_decode_and_attention_schedules(gpu, tmp_path):
    tuner = autotune.Autotuner(rounds=2, reps=4, cache=tmp_path / "t.json", stream_bytes=4 << 20)
    legal = [c["schedule"] for c in autotune.DecodeProblem(2, 4864, 896, stream_bytes=1 << 20).space()]
    assert tuner.decode_schedule(2, 4864, 896) in legal
    assert tuner.attention_schedule(130, 14, 2, 64) in range(5)
    assert tuner.rope_schedule(130, 1152, 896, 14, 2, 64) in (0, 16, 17, 20, 21, 24)
    again = autotune.Autotuner(cache=tmp_path / "t.json")
    assert again.decode_schedule(2, 4864, 896) == tuner.decode_schedule(2, 4864, 896)
    assert again.records[-1].cached


def test_tuned_model_decodes_the_default_tokens(gpu, tmp_path):
    """Qwen2.5-0.5B's widths (two layers) with every decode projection and the prompt's attention
    on tuned schedules: the same tokens, bit for bit the same logits, as the library's choices."""
    from dataclasses import replace

    from nanocompile_amd.models.config import QWEN25_05B, random_weights
    from nanocompile_amd.models.qwen2 import Qwen2
    config = replace(QWEN25_05B, num_hidden_layers=2)
    weights = random_weights(config, seed=21)
    prompt = [int(t) for t in np.random.default_rng(4).integers(0, config.vocab_size, 40)]
    tuner = autotune.Autotuner(rounds=2, reps=4, cache=tmp_path / "t.json", stream_bytes=4 << 20)
    tuned = Qwen2(config, weights, max_tokens=64, schedule=tuner)
    plain = Qwen2(config, weights, max_tokens=64)
    assert tuned.generate(prompt, 12) == plain.generate(prompt, 12)
    assert np.array_equal(tuned.forward(prompt).view(np.uint32), plain.forward(prompt).view(np.uint32))
    assert len(tuned.decode_schedules()) == 4
