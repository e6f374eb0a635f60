"""Stand-in graphs rebuilt from tests/golden/runner_graphs.json (the reference's own Qwen2 graphs,
recorded by tests/golden/make_runner_fixture.py): the attributes nanocompile_amd.runner reads."""

from __future__ import annotations

import json
from pathlib import Path
from types import SimpleNamespace

FIXTURE = Path(__file__).resolve().parent / "golden" / "runner_graphs.json"
MODE_OF = {"f32": "f32", "int8": "int8", "int8-vnni": "int8-vnni"}


def load() -> dict:
    return json.loads(FIXTURE.read_text())


class Dim:
    """A shape entry as the reference prints it (an int or a symbol name)."""

    def __init__(self, text: str) -> None:
        self.text = text

    def __str__(self) -> str:
        return self.text


def stand_in(desc: dict) -> SimpleNamespace:
    int8 = [json.loads(a) for a in desc["int8_attrs"]]
    nodes = []
    for op, count in desc["ops"].items():
        attrs = int8[0] if op in ("matmul_i8", "matmul_i8_vnni") and int8 else {}
        nodes += [SimpleNamespace(op=op, attrs=attrs) for _ in range(count)]
    return SimpleNamespace(
        name=desc["name"],
        inputs=[SimpleNamespace(attrs={"name": n}, dtype=t, shape=[Dim(d) for d in s])
                for n, t, s in desc["inputs"]],
        outputs={k: SimpleNamespace(dtype=t, shape=[Dim(d) for d in s]) for k, (t, s) in desc["outputs"].items()},
        weights={k: SimpleNamespace(dtype=t, shape=[Dim(d) for d in s]) for k, (t, s) in desc["weights"].items()},
        nodes=nodes,
    )
