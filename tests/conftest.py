"""Shared fixtures.

GPU tests are marked ``gpu`` and call the HIP library through its C ABI; the
rest run on any machine. The host C oracle is built on demand (gcc, about a
second) so a CPU-only run never depends on a previous build step; the HIP
library is only ever built by ``__graft_entry__.build()``.
"""

from __future__ import annotations

import numpy as np
import pytest


@pytest.fixture(scope="session")
def host():
    """The host C oracle library (oracle/nc_host.c), built if it is missing."""
    from oracle import build, host as H
    if not build.LIBRARY.exists():
        build.build()
    H.load()
    return H


@pytest.fixture(scope="session")
def gpu():
    """The HIP library bound to device 0. Raises (never skips) when it cannot be."""
    from nanocompile_amd import hip
    hip.init(0)
    return hip


def bits(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)
