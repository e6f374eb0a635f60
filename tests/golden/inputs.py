"""The seeded inputs the golden vectors were made from, regenerated without the reference.

make_golden.py (which runs the reference, in the build container only) and
the tests (anywhere, including the GPU machine, where the reference is absent)
both draw their inputs from here, so a fixture's inputs never have to be
stored; golden.json keeps their hashes to catch a changed generator.
"""

from __future__ import annotations

import numpy as np


def matmul_inputs(k: int, n: int, tokens: int, seed: int):
    """The reference test's projection inputs (test_int8.py:150-155): w N(0, 0.05), x N(0, 4), outliers x40."""
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((n, k)) * 0.05).astype(np.float32)
    x = (rng.standard_normal((tokens, k)) * 2).astype(np.float32)
    x[:, ::13] *= 40.0
    return w, x


def special_rows() -> np.ndarray:
    """The reference's quantizer special rows (test_int8.py:69-73)."""
    rng = np.random.default_rng(0)
    w = (rng.standard_normal((37, 70)) * 0.04).astype(np.float32)
    w[3] = 0.0
    w[5, :4] = [0.5, -0.5, 1.5, -2.5]
    w[5, 4] = 127.0 / 64
    return w
