"""The autotuner on the GPU: it measures, checks bits, caches, and the model runs on its choices."""

from __future__ import annotations

import numpy as np
import pytest

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
    assert {r.op for r in tuner.records} == {"matmul_i8_token", "matmul_i8_token_swiglu"}
    assert tuned.generate(list(ids[:8]), 6) == default.generate(list(ids[:8]), 6)
