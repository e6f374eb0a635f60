"""The whole tiny Qwen2 on the GPU against the reference's own compiled C (tests/golden G5).

make_golden.py ran the reference's Qwen2 through its C backend
(models/qwen2.py with CBackend) on a seeded tiny model in its float32 and two
int8 modes and recorded greedy tokens for four prompts, the logits of an
11-token prompt, and a decode step's logits. The GPU model in the same mode
must give the same greedy tokens and logits within 1e-4 of the largest logit:
its projections are the reference's kernels bit for bit (test_modes_gpu.py;
the float32 ones are the LM head's k-ordered kernel), and only the float
reductions around them (rms_norm's sum, the softmax) are summed in a tree
where the reference sums in index order.
"""

from __future__ import annotations

import hashlib
import json
from pathlib import Path

import numpy as np
import pytest

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"
PROMPTS = ([4, 5, 6], [7, 8], [1], [3, 1, 4, 1, 5, 9, 2, 6, 5, 3, 5])     # make_golden.py's G5 prompts
MODES = [("int8", "int8"), ("int8-vnni", "vnni"), ("f32", "f32")]
TOLERANCE = 1e-4          # max |ours - reference| over max |reference|, per logits array


@pytest.fixture(scope="module")
def golden():
    return np.load(GOLDEN / "golden.npz", allow_pickle=False)


@pytest.fixture(scope="module")
def weights():
    from nanocompile_amd.models.config import TINY, random_weights
    meta = json.loads((GOLDEN / "golden.json").read_text())["g5"]
    w = random_weights(TINY, seed=meta["seed"], std=meta["std"])
    for name, digest in meta["weights_sha"].items():
        assert hashlib.sha256(np.ascontiguousarray(w[name]).tobytes()).hexdigest()[:16] == digest, name
    return w


@pytest.fixture(scope="module", params=MODES, ids=[m for m, _ in MODES])
def model(gpu, weights, request):
    from nanocompile_amd.models.config import TINY
    from nanocompile_amd.models.qwen2 import Qwen2
    mode, tag = request.param
    return Qwen2(TINY, weights, quantization=mode, max_tokens=64), tag


def close(ours, reference):
    ours, reference = np.asarray(ours, np.float64), np.asarray(reference, np.float64)
    return np.max(np.abs(ours - reference)) / np.max(np.abs(reference))


def test_greedy_tokens_are_the_references(model, golden):
    from nanocompile_amd.models.qwen2 import greedy
    m, tag = model
    print(f"G5 greedy {tag}", flush=True)
    for i, prompt in enumerate(PROMPTS):
        assert greedy(m, prompt, 8) == [int(t) for t in golden[f"g5_{tag}_tokens_{i}"]], (tag, i)
        assert m.generate(prompt, 8) == [int(t) for t in golden[f"g5_{tag}_tokens_{i}"]], (tag, i)


def test_logits_are_the_references(model, golden):
    m, tag = model
    ids = np.array(PROMPTS[3])
    rel = close(m.forward(ids, m.new_cache(16)), golden[f"g5_{tag}_logits"])
    print(f"G5 logits {tag}: {rel:.2e}", flush=True)
    assert rel <= TOLERANCE
    cache = m.new_cache(16)
    m.forward(ids[:6], cache)
    rel = close(m.forward(ids[6:7], cache, last_only=True), golden[f"g5_{tag}_decode_logits"])
    assert rel <= TOLERANCE


def test_the_modes_differ_from_each_other(model, golden):
    """The fixture holds distinct results per mode, so passing above is not a coincidence of modes."""
    _, tag = model
    for other in {"int8", "vnni", "f32"} - {tag}:
        assert close(golden[f"g5_{other}_logits"], golden[f"g5_{tag}_logits"]) > 10 * TOLERANCE
