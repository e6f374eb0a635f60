"""Builds the host C oracle/baseline into ``oracle/_lib/libnc_host.so``. TEST INFRASTRUCTURE.

Flags as the reference builds its generated C (codegen_c.py:50) minus
``-march=native``: the ISA-specific loops carry their own target attributes
and are chosen at run time, so the library built here runs on any x86-64
host, including the GPU box's, whose CPU is not known in advance.
"""

from __future__ import annotations

import os
import shutil
import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
LIB_DIR = HERE / "_lib"
LIBRARY = LIB_DIR / "libnc_host.so"
CFLAGS = ("-O3", "-ffp-contract=off", "-fwrapv", "-fno-math-errno", "-fPIC", "-shared", "-pthread",
          "-fvisibility=hidden", "-std=gnu11")


def build(verbose: bool = False) -> Path:
    cc = os.environ.get("CC") or shutil.which("gcc") or "cc"
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    scratch = LIBRARY.with_suffix(".so.tmp")
    cmd = [cc, *CFLAGS, "-o", str(scratch), str(HERE / "nc_host.c"), str(HERE / "nc_model.c"), str(HERE / "nc_modes.c"), "-lm"]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"gcc failed on nc_host.c:\n{result.stderr[-6000:]}")
    os.replace(scratch, LIBRARY)
    if verbose:
        print(f"built {LIBRARY}")
    return LIBRARY


if __name__ == "__main__":
    build(verbose=True)
