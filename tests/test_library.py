"""The C ABI: the HIP library loads on any machine and exports what include/nc_hip.h declares.

No kernel is called here (that needs a GPU); loading the library and
resolving its symbols does not touch the device.
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "nc_hip.h"


def declared() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return re.findall(r"^\s*[\w\s\*]+?\b(nc_\w+)\s*\(", text, flags=re.M)


@pytest.fixture(scope="module")
def library():
    from nanocompile_amd import build
    if not build.LIBRARY.exists():
        build.build()
    return ctypes.CDLL(str(build.LIBRARY))


def test_the_header_declares_the_entry_points():
    names = declared()
    assert "nc_matmul_i8_token" in names and "nc_sync" in names and len(names) == len(set(names))


def test_every_declared_symbol_is_exported(library):
    missing = [name for name in declared() if not hasattr(library, name)]
    assert not missing, missing


def test_kernel_entry_points_have_the_reference_calling_convention():
    """int32_t nc_x(void **p, const int64_t *s) for every kernel (codegen_c.py:5-10)."""
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    kernels = re.findall(r"int32_t (nc_\w+)\(void \*\*p, const int64_t \*s\);", text)
    assert "nc_matmul_i8_token" in kernels and "nc_rms_norm_quant" in kernels


def test_the_product_never_imports_the_oracle():
    """nanocompile_amd has no CPU fallback: no module of it imports oracle/."""
    import ast
    for path in (ROOT / "nanocompile_amd").rglob("*.py"):
        tree = ast.parse(path.read_text())
        for node in ast.walk(tree):
            names = []
            if isinstance(node, ast.Import):
                names = [a.name for a in node.names]
            elif isinstance(node, ast.ImportFrom):
                names = [node.module or ""]
            assert not any(n == "oracle" or n.startswith("oracle.") for n in names), path
