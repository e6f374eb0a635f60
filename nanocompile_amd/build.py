"""Building the HIP library: every ``csrc/*.hip`` for gfx950, linked into one ``.so``.

The library lands in ``nanocompile_amd/_lib/libnc_hip.so``, inside the package,
so it travels with the source tree to the machine that runs it; nothing is
installed anywhere else. The reference builds its generated C the same way,
with a fixed flag set that forbids the compiler from changing what the code
computes (codegen_c.py:16-22, 50): here ``-ffp-contract=off`` stops hipcc
(which contracts by default) from fusing a multiply and an add, and the
kernels spell out correctly rounded division and square root themselves.
"""

from __future__ import annotations

import hashlib
import os
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
CSRC = PACKAGE / "csrc"
LIB_DIR = PACKAGE / "_lib"
OBJ_DIR = PACKAGE / "_lib" / "obj"
LIBRARY = LIB_DIR / "libnc_hip.so"
ARCH = "gfx950"

HIPCC_FLAGS = (
    "-O3", "-std=c++17", f"--offload-arch={ARCH}", "-fPIC", "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-fvisibility=hidden", "-munsafe-fp-atomics",
    # Packed fp32 instructions have given wrong results on these machines:
    # hipcc must not form them from ordinary float code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
)


class BuildError(RuntimeError):
    """hipcc rejected a source file."""


def hipcc() -> str:
    path = os.environ.get("HIPCC") or shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists() and shutil.which(path) is None:
        raise BuildError("hipcc not found: install ROCm or set HIPCC")
    return path


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def library_digest() -> str:
    """A hash of every kernel source and header and the flags: the library's version.

    Compiled into the library (``nc_library_digest``) so that what was measured
    on one build (tuning winners) is not reused on another.
    """
    h = hashlib.sha256("\0".join(HIPCC_FLAGS).encode())
    for path in sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.h")):
        h.update(path.name.encode() + b"\0" + path.read_bytes())
    return h.hexdigest()[:16]


def _compile(src: Path, digest: str) -> Path:
    obj = OBJ_DIR / (src.stem + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, f"-I{CSRC}", f'-DNC_LIBRARY_DIGEST="{digest}"', "-c", str(src), "-o", str(obj)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise BuildError(f"hipcc failed on {src.name}:\n{result.stderr[-6000:]}")
    return obj


def build(jobs: int | None = None, verbose: bool = False) -> Path:
    """Compile every source and link the library; returns its path."""
    OBJ_DIR.mkdir(parents=True, exist_ok=True)
    srcs = sources()
    jobs = jobs or min(len(srcs), os.cpu_count() or 4, 16)
    digest = library_digest()
    with ThreadPoolExecutor(max_workers=max(1, jobs)) as pool:
        objs = list(pool.map(lambda src: _compile(src, digest), srcs))
    scratch = LIBRARY.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(scratch), *map(str, objs)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise BuildError(f"linking {LIBRARY.name} failed:\n{result.stderr[-6000:]}")
    os.replace(scratch, LIBRARY)
    if verbose:
        print(f"built {LIBRARY} from {len(srcs)} sources")
    return LIBRARY


if __name__ == "__main__":
    build(verbose=True)
