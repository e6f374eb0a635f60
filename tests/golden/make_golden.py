"""Writes the golden vectors in this directory by running the reference itself.

Run in the build container only, where /root/reference (SpookyJumpyBeans/
nanocompile) is mounted:

    python tests/golden/make_golden.py

(the reference's compile cache goes to a fresh temporary directory unless
NANOCOMPILE_CACHE names one)

It imports the reference's package from /root/reference, builds small graphs
with its own frontend, compiles them with its own C code generator (gcc), and
records the outputs. Nothing of the reference is copied: the fixtures are
inputs (or the seeds that make them, with a hash to catch a changed generator)
and the reference's outputs. The reference never travels to the GPU machine;
these files do.

What each group pins (the oracle cannot pin these by itself):
  G1  quantize_int8 (quantize.py:55-70) on the special rows and a seeded
      [4864, 896] matrix
  G2  matmul_i8 in the reference's generated C: the 32-chain FMA order of
      lower.py:294-356, unfused, fused and scheduled
  G3  matmul_i8_vnni (block 32): the Dp4 / block-scale order of
      lower.py:359-397, and the block activation quantizer of
      quantize.py:102-124
  G4  fused row and elementwise kernels: rms_norm, softmax with the causal
      mask, silu(gate) * up, RoPE, and the inverse frequencies (nn.py)
  G5  a seeded tiny Qwen2 (models/qwen2.py): greedy tokens and logits in
      float32, int8 and int8-vnni, interpreter and generated C
"""

from __future__ import annotations

import hashlib
import json
import os
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
# The reference compiles its generated C into a cache directory; keep it out of the repository.
os.environ.setdefault("NANOCOMPILE_CACHE", tempfile.mkdtemp(prefix="nanocompile-cache-"))

from nanocompile import dtypes, interpreter, nn, quantize  # noqa: E402  (the reference)
from nanocompile.frontend import GraphBuilder  # noqa: E402
from nanocompile.models.qwen2 import Qwen2, Qwen2Config, greedy  # noqa: E402
from nanocompile.runtime import CBackend, CompiledGraph  # noqa: E402

from nanocompile_amd.models import config as ours  # noqa: E402  (the seeded weight generator)
from tests.golden.inputs import matmul_inputs, special_rows  # noqa: E402


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()[:16]


OUT: dict[str, np.ndarray] = {}
META: dict[str, object] = {}


def put(name: str, a) -> None:
    OUT[name] = np.ascontiguousarray(a)


# -- G1: the weight quantizer ------------------------------------------------------


def g1() -> None:
    values, scales = quantize.quantize_int8(special_rows())
    put("g1_special_values", values)
    put("g1_special_scales", scales)
    w = (np.random.default_rng(1).standard_normal((4864, 896)) * 0.02).astype(np.float32)
    values, scales = quantize.quantize_int8(w)
    META["g1_big"] = {"w_sha": sha(w), "values_sha": sha(values), "scales_sha": sha(scales)}
    put("g1_big_values_head", values[:4])
    put("g1_big_scales", scales)


# -- G2 / G3: the two int8 matmuls --------------------------------------------------

WIDTHS = [(896, 72), (4864, 24), (77, 40), (40, 16), (160, 40), (96, 24)]
TOKENS = [1, 3, 7]


def projection(k: int, n: int):
    b = GraphBuilder("projection")
    x = b.input("x", dtypes.f32, (b.symbol("seq"), k))
    return b.build({"y": nn.linear(x, b.weight("w", (n, k)))})


def g2_g3() -> None:
    for activations, tag in (("f32", "g2"), ("int8", "g3")):
        for k, n in WIDTHS:
            if activations == "int8" and k % quantize.DEFAULT_BLOCK:
                continue
            graph = quantize.quantize(projection(k, n), activations)
            compiled = [CompiledGraph(graph, **o) for o in ({"fuse": False}, {"schedule": None}, {})]
            for tokens in TOKENS:
                w, x = matmul_inputs(k, n, tokens, seed=k + tokens)
                weights = quantize.quantized_weights(graph, {"w": w})
                outs = [c({"x": x}, weights)["y"] for c in compiled]
                for o in outs[1:]:
                    assert np.array_equal(o.view(np.uint32), outs[0].view(np.uint32)), (tag, k, n, tokens)
                key = f"{tag}_{k}_{n}_{tokens}"
                put(key, outs[0])
                put(key + "_interp", interpreter.run(graph, {"x": x}, weights)["y"])
                META[key] = {"w_sha": sha(w), "x_sha": sha(x)}


def g3_quantizer() -> None:
    """The block activation quantizer as the reference's graph ops compute it (C and interpreter)."""
    b = GraphBuilder("blocks")
    x = b.input("x", dtypes.f32, (b.symbol("seq"), 96))
    xq, xs, offset = quantize.quantize_activations(x.node, 32)
    from nanocompile.frontend import Tensor
    graph = b.build({"xq": Tensor(xq, b), "xs": Tensor(xs, b), "offset": Tensor(offset, b)})
    _, xv = matmul_inputs(96, 1, 5, seed=96 + 5)
    got = CompiledGraph(graph)({"x": xv}, {})
    for name in ("xq", "xs", "offset"):
        put(f"g3_quant_{name}", got[name])
    META["g3_quant"] = {"x_sha": sha(xv)}


# -- G4: fused groups ------------------------------------------------------------------


def run_c_and_interp(graph, inputs, weights, key):
    c = CompiledGraph(graph)(inputs, weights)
    i = interpreter.run(graph, inputs, weights)
    for name in c:
        put(f"{key}_{name}", c[name])
        put(f"{key}_{name}_interp", i[name])


def g4() -> None:
    rng = np.random.default_rng(40)
    # rms_norm, the model's width
    b = GraphBuilder("rms")
    x = b.input("x", dtypes.f32, (b.symbol("seq"), 896))
    graph = b.build({"y": nn.rms_norm(x, b.weight("w", (896,)), 1e-6)})
    xv = rng.standard_normal((3, 896)).astype(np.float32)
    xv[rng.random(xv.shape) < 0.01] *= 20
    wv = (1 + 0.1 * rng.standard_normal(896)).astype(np.float32)
    put("g4_rms_x", xv)
    put("g4_rms_w", wv)
    run_c_and_interp(graph, {"x": xv}, {"w": wv}, "g4_rms")

    # softmax(scores + causal mask) over [heads, seq, past + seq]
    b = GraphBuilder("softmax")
    seq, past = b.symbol("seq"), b.symbol("past")
    s = b.input("s", dtypes.f32, (4, seq, past + seq))
    b.input("p", dtypes.f32, (past,))          # binds past
    graph_inputs = None
    mask = nn.causal_mask(b, seq, past)
    graph = b.build({"y": nn.softmax(s + mask, axis=-1)})
    for seq_v, past_v in ((1, 12), (5, 3)):
        sv = (rng.standard_normal((4, seq_v, past_v + seq_v)) * 3).astype(np.float32)
        key = f"g4_softmax_{seq_v}_{past_v}"
        put(key + "_s", sv)
        run_c_and_interp(graph, {"s": sv, "p": np.zeros(past_v, np.float32)}, {}, key)
    del graph_inputs

    # silu(gate) * up
    b = GraphBuilder("swiglu")
    g = b.input("g", dtypes.f32, (b.symbol("seq"), 64))
    u = b.input("u", dtypes.f32, (b.symbol("seq"), 64))
    graph = b.build({"y": nn.silu(g) * u})
    gv = (rng.standard_normal((3, 64)) * 30).astype(np.float32)
    gv[0, :4] = 0.0
    uv = rng.standard_normal((3, 64)).astype(np.float32)
    put("g4_silu_g", gv)
    put("g4_silu_u", uv)
    run_c_and_interp(graph, {"g": gv, "u": uv}, {}, "g4_silu")

    # RoPE on [heads, seq, 64] at positions past .. past + seq - 1, theta 1e6
    b = GraphBuilder("rope")
    seq, past = b.symbol("seq"), b.symbol("past")
    xr = b.input("x", dtypes.f32, (3, seq, 64))
    b.input("p", dtypes.f32, (past,))
    positions = b.iota((seq,), axis=0) + b.dim(past)
    cos, sin = nn.rope_tables(positions, 64, 1e6)
    graph = b.build({"y": nn.apply_rope(xr, cos, sin)})
    for seq_v, past_v in ((1, 511), (7, 0), (2, 100000)):
        xv = rng.standard_normal((3, seq_v, 64)).astype(np.float32)
        key = f"g4_rope_{seq_v}_{past_v}"
        put(key + "_x", xv)
        run_c_and_interp(graph, {"x": xv, "p": np.zeros(past_v, np.float32)}, {}, key)
    put("g4_inv_freq_64_1e6", nn.inverse_frequencies(64, 1e6))
    put("g4_inv_freq_32_1e6", nn.inverse_frequencies(32, 1e6))


# -- G5: a tiny model ------------------------------------------------------------------

PROMPTS = ([4, 5, 6], [7, 8], [1], [3, 1, 4, 1, 5, 9, 2, 6, 5, 3, 5])


def g5() -> None:
    c = ours.TINY
    config = Qwen2Config(c.vocab_size, c.hidden_size, c.intermediate_size, c.num_hidden_layers,
                         c.num_attention_heads, c.num_key_value_heads, c.rms_norm_eps, c.rope_theta,
                         c.tie_word_embeddings)
    weights = ours.random_weights(c, seed=5, std=ours.TINY_STD)
    META["g5"] = {"weights_sha": {k: sha(v) for k, v in list(weights.items())[:3]}, "seed": 5,
                  "std": ours.TINY_STD}
    for mode in (None, "int8", "int8-vnni"):
        tag = {None: "f32", "int8": "int8", "int8-vnni": "vnni"}[mode]
        model = Qwen2(config, weights, run=CBackend(), quantization=mode)
        interp = Qwen2(config, weights, quantization=mode)
        for i, prompt in enumerate(PROMPTS):
            put(f"g5_{tag}_tokens_{i}", np.array(greedy(model, prompt, 8), np.int64))
        ids = np.array(PROMPTS[3])
        put(f"g5_{tag}_logits", model.forward(ids))
        put(f"g5_{tag}_logits_interp", interp.forward(ids))
        cache = model.new_cache(16)
        model.forward(ids[:6], cache=cache)
        put(f"g5_{tag}_decode_logits", model.forward(ids[6:7], cache=cache, last_only=True))


def main() -> None:
    started = time.time()
    g1()
    g2_g3()
    g3_quantizer()
    g4()
    g5()
    META["numpy"] = np.__version__
    META["reference"] = str(REFERENCE)
    np.savez_compressed(HERE / "golden.npz", **OUT)
    (HERE / "golden.json").write_text(json.dumps(META, indent=1, sort_keys=True))
    size = (HERE / "golden.npz").stat().st_size
    print(f"wrote {len(OUT)} arrays ({size / 1024:.0f} KiB) in {time.time() - started:.0f} s")


if __name__ == "__main__":
    main()
