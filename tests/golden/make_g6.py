"""Writes g6.json and g6.npz: the reference's own run of config 5's workload, in its two int8 modes.

Run in the build container only, where /root/reference is mounted:

    python tests/golden/make_g6.py

The workload is exactly the one bench.py times and tests/test_configs_gpu.py
checks: the Qwen2.5-0.5B-shaped model (24 layers, vocabulary 151,936) with
``random_weights(QWEN25_05B, seed=0)`` and a 128-token prompt drawn from
``default_rng(1)``. The reference builds it as ``Qwen2(config, weights,
run=CBackend(), quantization=mode)`` (models/qwen2.py:274-311, its compiled C,
runtime.py:321-337) for ``mode`` in ``int8`` (fp32 activations times int8
weights, the 32-chain order) and ``int8-vnni`` (int8 activations in blocks of
32, the Dp4 order), and decodes greedily with its own ``greedy``
(models/qwen2.py:348-368) for 257 new tokens: the prompt's call, then 256
one-token calls at cache lengths 128 ... 383.

Recorded per mode: the 257 tokens; for the calls at cache length 0 (the
prompt), 255 and 383, the argmax, the largest logit, and the logits at every
97th vocabulary entry. A recording wrapper around the reference's runner keeps
each call's logits; nothing of the reference is copied, only its outputs.

``--math nc`` records the same runs again, under the tags ``int8_ncmath`` and
``vnni_ncmath``, with the reference's compiled C calling this package's expf,
sinf and cosf (csrc/nc_math.h, the functions the GPU kernels use) in place of
the C library's: nc_math_shim.c is built with gcc and preloaded into a child
process. The int8-vnni mode rounds its activations to int8 at every
projection, so a last-bit difference anywhere moves roundings downstream: the
reference's own logits move by 2.1% of the largest when every norm weight
moves by one ulp, and by 2.4% between the C library's functions and these
(their results differ in the last bit on a small fraction of inputs). With the
same functions on both sides the whole model can be held bit for bit.
"""

from __future__ import annotations

import ctypes
import json
import os
import subprocess
import sys
import tempfile
import time
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
REFERENCE = Path(os.environ.get("NANOCOMPILE_REFERENCE", "/root/reference"))
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(REFERENCE))
os.environ.setdefault("NANOCOMPILE_CACHE", tempfile.mkdtemp(prefix="nanocompile-cache-"))

from nanocompile.models.qwen2 import Qwen2, Qwen2Config, greedy  # noqa: E402  (the reference)
from nanocompile.runtime import CBackend  # noqa: E402

from nanocompile_amd.models import config as ours  # noqa: E402  (the seeded weight generator)

SEED, PROMPT, NEW = 0, 128, 257          # bench.py's weights seed; the prompt draws from SEED + 1
STRIDE = 97                              # logits kept at every 97th vocabulary entry
CHECKED = {0: 0, 255: 128, 383: 256}     # cache length before the call -> index of the call


class Recording:
    """A Runner (models/qwen2.py:229) that keeps the last row of every call's logits."""

    def __init__(self, run) -> None:
        self.run = run
        self.logits: list[np.ndarray] = []

    def __call__(self, graph, inputs, weights):
        out = self.run(graph, inputs, weights)
        self.logits.append(np.array(out["logits"][-1], np.float32, copy=True))
        return out


def preloaded_math() -> bool:
    """Whether nc_math_shim.c's functions are the process's expf, sinf and cosf."""
    return hasattr(ctypes.CDLL(None), "nc_g6_math_shim")


def rerun_with_nc_math(modes: list[str]) -> None:
    """Build nc_math_shim.c and run this script again with it preloaded."""
    with tempfile.TemporaryDirectory() as scratch:
        shim = Path(scratch) / "nc_math_shim.so"
        subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-fPIC", "-shared", "-o", str(shim),
                        str(HERE / "nc_math_shim.c"), "-lm"], check=True)
        env = dict(os.environ, LD_PRELOAD=str(shim))
        subprocess.run([sys.executable, __file__, "--math", "nc", *modes], env=env, check=True)


def main() -> None:
    args = sys.argv[1:]
    nc_math = args[:2] == ["--math", "nc"]
    if nc_math:
        args = args[2:]
        if not preloaded_math():
            rerun_with_nc_math(args)
            return
    c = ours.QWEN25_05B
    config = Qwen2Config(c.vocab_size, c.hidden_size, c.intermediate_size, c.num_hidden_layers,
                         c.num_attention_heads, c.num_key_value_heads, c.rms_norm_eps, c.rope_theta,
                         c.tie_word_embeddings)
    weights = ours.random_weights(c, seed=SEED)
    prompt = [int(t) for t in np.random.default_rng(SEED + 1).integers(0, c.vocab_size, PROMPT)]
    meta: dict[str, object] = {"seed": SEED, "prompt_seed": SEED + 1, "prompt": prompt, "new_tokens": NEW,
                               "stride": STRIDE, "checked_past": sorted(CHECKED)}
    arrays: dict[str, np.ndarray] = {}
    modes = args or ["int8", "int8-vnni"]
    for mode in modes:
        tag = {"int8": "int8", "int8-vnni": "vnni"}[mode] + ("_ncmath" if nc_math else "")
        recorder = Recording(CBackend())
        model = Qwen2(config, weights, run=recorder, quantization=mode)
        start = time.time()
        tokens = greedy(model, prompt, NEW)
        print(f"{mode}: {NEW} tokens in {time.time() - start:.0f} s: {tokens[:8]} ...", flush=True)
        assert len(recorder.logits) == NEW
        entry: dict[str, object] = {"tokens": tokens}
        for past, call in CHECKED.items():
            logits = recorder.logits[call]
            assert int(np.argmax(logits)) == tokens[call]
            entry[f"argmax_{past}"] = int(np.argmax(logits))
            entry[f"max_{past}"] = float(np.max(logits)).hex()
            arrays[f"{tag}_logits_{past}"] = np.ascontiguousarray(logits[::STRIDE])
        meta[tag] = entry
    old_meta = json.loads((HERE / "g6.json").read_text()) if (HERE / "g6.json").exists() else {}
    old_meta.update(meta)
    (HERE / "g6.json").write_text(json.dumps(old_meta, indent=1, sort_keys=True) + "\n")
    if (HERE / "g6.npz").exists():
        with np.load(HERE / "g6.npz", allow_pickle=False) as old:
            arrays = {**{k: old[k] for k in old.files}, **arrays}
    np.savez_compressed(HERE / "g6.npz", **arrays)
    print(f"wrote g6.json and g6.npz ({len(arrays)} arrays)")


if __name__ == "__main__":
    main()
