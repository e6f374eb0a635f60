"""Qwen2 on the HIP kernels: the reference's model driver (models/qwen2.py), MI355X-side.

The reference compiles one graph over (seq, past) and runs it a kernel call at
a time from Python, with the KV cache in host memory (models/qwen2.py:167-345,
runtime.py:245-301). Here the same forward pass is a fixed sequence of HIP
kernels per layer, the weights and the KV cache live on the device, and the
driver only uploads token ids and downloads what the caller asks for:

    rms_norm + per-token int8 ......... nc_rms_norm_quant
    q, k, v projections + bias ........ nc_matmul_i8_token (rows concatenated)
    RoPE, cache append ................ nc_rope_append
    attention (GQA, causal), and the
    per-token int8 of the context ..... nc_attention
    o projection + residual ........... nc_matmul_i8_token (in place on x)
    rms_norm + per-token int8 ......... nc_rms_norm_quant
    gate, up, silu(gate) * up ......... nc_matmul_i8_token_swiglu
    per-token int8 of h ............... nc_quantize_token_i8
    down projection + residual ........ nc_matmul_i8_token (in place on x)

then the final rms_norm, the float32 tied LM head (the reference keeps it
float32, quantize.py:24-28) and the argmax. ``quantization="int8-token"`` is
the north star's mode: per-row int8 weights, per-token int8 activations,
exact int32 accumulation. ``"int8"`` and ``"int8-vnni"`` are the reference's
own modes (quantize.py:127-164): float32 activations times int8 weights in
its 32-chain order, or 32-wide int8 activation blocks in its VNNI order, each
bit for bit with its generated C (nc_matmul_i8, nc_matmul_i8_vnni). ``"f32"``
is the reference's float32 model (``quantization=None``): every projection
is its float32 matmul kernel's order (k in order, multiply then add, then +
bias), which is the LM head's kernel over a packed table (nc_lm_head).

Memory: one device arena per model (one hipMalloc, made once): the weights,
then the activations for up to ``max_tokens`` new tokens; and one per sequence
(``new_cache``, the caller's, as the reference's KVCache is): keys, values,
RoPE's table, attention's workspace and a device-driven decode's token
history and position. A decode step moves nothing but a token id in and
(optionally) a row of logits out. (A checkpoint with an untied LM head is
uploaded once more, temporarily, to be packed.)
"""

from __future__ import annotations

from collections.abc import Mapping, Sequence

import numpy as np

from nanocompile_amd import hip
from nanocompile_amd.hip import DeviceArray
from nanocompile_amd.kernels import (MAX_KEYS, argmax_slots, attention_workspace_bytes, float_bits, pack_chains,
                                     pack_chains_vnni)
from nanocompile_amd.models.config import Qwen2Config

QUANTIZATIONS = ("int8-token", "int8", "int8-vnni", "f32")
BLOCK = 32          # matmul_i8_vnni's activation block (quantize.py:44)
ALIGN = 256


def _packed_bytes(quantization: str, n: int, k: int) -> int:
    """Bytes of pack_chains (int8) or pack_chains_vnni (int8-vnni) of an [n, k] weight."""
    if quantization == "int8":
        return n * -(-(k // 32) // 4) * 128
    return n * (k // 128) * 128


WORKSPACE_BYTES = 64 << 20     # attention chunk results held at once (longer prompts go in slabs)
REFERENCE_ORDER_KEYS = 16000   # nc_attention_index_order: a float of LDS per position


def inverse_frequencies(head_dim: int, theta: float) -> np.ndarray:
    """RoPE's per-plane rates in float32, as the reference computes them (nn.py:69-75)."""
    exponent = np.arange(0, head_dim, 2, dtype=np.int64).astype(np.float32) / np.float32(head_dim)
    return (np.float32(1.0) / (np.float32(theta) ** exponent)).astype(np.float32)


class Arena:
    """One device allocation carved into aligned arrays (the reference's arena, runtime.py:39, 97-143)."""

    def __init__(self, nbytes: int) -> None:
        self.base = DeviceArray((max(1, nbytes),), np.uint8)
        self.top = 0

    @staticmethod
    def size(shapes: Sequence[tuple[tuple[int, ...], np.dtype]]) -> int:
        total = 0
        for shape, dtype in shapes:
            total += -(-int(np.prod(shape, dtype=np.int64)) * np.dtype(dtype).itemsize // ALIGN) * ALIGN
        return total

    def take(self, shape, dtype) -> DeviceArray:
        nbytes = int(np.prod(shape, dtype=np.int64)) * np.dtype(dtype).itemsize
        view = self.base.view(shape, dtype, offset_bytes=self.top)
        self.top += -(-nbytes // ALIGN) * ALIGN
        return view


def _rope_schedule_ok(schedule: int, head_dim: int) -> bool:
    """Whether nc_matmul_i8_token_rope can run ``schedule``: its own choice (0) or an MFMA tile
    whose n is one head."""
    if schedule == 0:
        return True
    shape = hip.schedule_info(schedule) if schedule >= 16 else None
    return shape is not None and shape.get("tile_n") == head_dim


class KVCache:
    """Keys and values of one sequence on the device: ``[layers, kv_heads, capacity, head_dim]`` each.

    The reference grows its host cache by doubling (models/qwen2.py:232-271);
    on the device the capacity is fixed when the cache is made, since 288 GB
    of HBM leaves room to size it for the whole sequence up front.
    """

    def __init__(self, config: Qwen2Config, capacity: int = 256) -> None:
        if not 0 < capacity <= MAX_KEYS:
            raise ValueError(f"capacity {capacity}: a cache holds 1 to {MAX_KEYS} tokens (the attention "
                             f"kernels' limit on keys)")
        self.config, self.capacity, self.length = config, capacity, 0
        shape = (config.num_hidden_layers, config.num_key_value_heads, capacity, config.head_dim)
        D = config.head_dim
        # attention's chunk results (nc_attention, nc_attention_decode): every
        # query row of a prompt up to 64 MiB, longer prompts in slabs
        per_row = attention_workspace_bytes(config.num_attention_heads, D, 1, capacity)
        self.work_bytes = per_row * max(1, min(capacity, WORKSPACE_BYTES // per_row))
        # One hipMalloc for the sequence: keys, values, RoPE's table, the attention
        # workspace, and a device-driven decode's token history and position.
        parts = [(shape, np.float32), (shape, np.float32), ((2, capacity, D // 2), np.float32),
                 ((self.work_bytes // 4,), np.float32), ((capacity,), np.int64), ((1,), np.int64),
                 ((D // 2,), np.float32)]
        self.arena = Arena(Arena.size(parts))
        self.keys, self.values = self.arena.take(shape, np.float32), self.arena.take(shape, np.float32)
        self._layer = config.num_key_value_heads * capacity * D * 4
        # cos and sin of every position's RoPE angles (nc_rope_table), for the
        # decode attention kernel: the same bits it would compute, one lookup
        self.rope = self.arena.take((2, capacity, D // 2), np.float32)
        self.work = self.arena.take((self.work_bytes // 4,), np.float32)
        self.tokens, self.position = self.arena.take((capacity,), np.int64), self.arena.take((1,), np.int64)
        inv = self.arena.take((D // 2,), np.float32)
        inv.upload(inverse_frequencies(D, config.rope_theta))
        hip.call("nc_rope_table", [self.rope, inv], [capacity, D])
        hip.sync()

    def layer(self, index: int) -> tuple[int, int]:
        return self.keys.ptr + index * self._layer, self.values.ptr + index * self._layer

    def past(self) -> tuple[np.ndarray, np.ndarray]:
        """The filled part, copied to the host (the reference's ``KVCache.past``)."""
        return self.keys.numpy()[:, :, : self.length], self.values.numpy()[:, :, : self.length]


class Qwen2:
    """The model's front door on the GPU: token ids in, logits out (models/qwen2.py:278-345)."""

    def __init__(self, config: Qwen2Config, weights: Mapping[str, np.ndarray], quantization: str = "int8-token",
                 max_tokens: int = 512, device: int = 0, schedule="default") -> None:
        """``schedule`` picks the projections' launch shapes, as the reference's
        ``CompiledGraph(schedule=...)`` does (runtime.py:167-222): "default" (or
        None) for the library's choice, or an ``autotune.Autotuner``, which
        measures each projection shape on first use and caches the winner."""
        if quantization not in QUANTIZATIONS:
            raise ValueError(f"quantization must be one of {QUANTIZATIONS}")
        if schedule not in ("default", None) and not hasattr(schedule, "schedule"):
            raise ValueError("schedule must be 'default', None or an autotune.Autotuner")
        hip.init(device)
        self.config, self.quantization, self.max_tokens = config, quantization, max_tokens
        self.tuner = None if schedule in ("default", None) else schedule
        c = config
        H, I, D = c.hidden_size, c.intermediate_size, c.head_dim
        Q, KVW = c.num_attention_heads * D, c.num_key_value_heads * D
        W = Q + 2 * KVW
        self.width = W
        L, V = c.num_hidden_layers, c.vocab_size
        if H % 4 or H % 16 or I % 16:
            raise ValueError("hidden and intermediate sizes must be multiples of 16")
        vblocks = -(-V // 64) * 64

        pad = lambda n: -(-n // 64) * 64       # rows of a packed float32 table (nc_pack_rows64)
        if quantization == "f32":              # the reference's float32 model: packed f32 projections
            per_layer = [((H,), np.float32), ((H,), np.float32), ((pad(W), H), np.float32), ((W,), np.float32),
                         ((pad(H), Q), np.float32), ((pad(I), H), np.float32), ((pad(I), H), np.float32),
                         ((pad(H), I), np.float32)]
        else:
            per_layer = [((H,), np.float32), ((H,), np.float32), ((W, H), np.int8), ((W,), np.float32),
                         ((W,), np.float32), ((H, Q), np.int8), ((H,), np.float32), ((I, H), np.int8),
                         ((I,), np.float32), ((I, H), np.int8), ((I,), np.float32), ((H, I), np.int8),
                         ((H,), np.float32)]
        if quantization in ("int8", "int8-vnni"):   # the reference modes' packed copies (pack_chains*)
            per_layer += [((_packed_bytes(quantization, n, k),), np.int8)
                          for n, k in ((W, H), (H, Q), (I, H), (I, H), (H, I))]
        shapes = per_layer * L + [((V, H), np.float32), ((vblocks, H), np.float32), ((H,), np.float32),
                                  ((D // 2,), np.float32)]
        M = max_tokens
        act = [((M, H), np.float32), ((M, W), np.float32), ((M, Q), np.float32), ((M, I), np.float32),
               ((M, max(I, H, Q)), np.int8), ((M,), np.float32), ((M, H), np.float32), ((M,), np.int64),
               ((argmax_slots(V),), np.uint64), ((1, V), np.float32), ((M,), np.int64), ((M, I), np.float32),
               ((M, I), np.float32), ((M, -(-max(I, H, Q) // BLOCK)), np.float32), ((M,), np.float32)]
        # One hipMalloc: the weights, then the activations. While the weights load, the
        # activation region (not yet in use) holds the float32 rows being quantized.
        stage_floats = max(I * H, W * H, H * Q)
        weight_bytes = Arena.size(shapes)
        self.arena = Arena(weight_bytes + max(Arena.size(act), Arena.size([((stage_floats,), np.float32)])))
        self.weights = self.arena
        stage = self.arena.base.view((stage_floats,), np.float32, offset_bytes=weight_bytes)

        def upload(name: str, into: DeviceArray) -> DeviceArray:
            into.upload(np.ascontiguousarray(weights[name], np.float32))
            return into

        def quantized(names: Sequence[str], rows: int, k: int) -> tuple:
            """Per-row int8 of the named matrices stacked row-wise (quantize.py:55-70, on the device),
            plus, for the reference's modes, the packed copy their kernels read (made once); in the
            float32 mode, (None, None, the stacked float32 rows packed as nc_lm_head reads them)."""
            if quantization == "f32":
                at = 0
                for name in names:
                    w = np.ascontiguousarray(weights[name], np.float32)
                    if w.shape[1] != k:
                        raise ValueError(f"{name} has width {w.shape[1]}, expected {k}")
                    stage.view(w.shape, np.float32, offset_bytes=at * k * 4).upload(w)
                    at += w.shape[0]
                if at != rows:
                    raise ValueError(f"{names} have {at} rows, expected {rows}")
                packed = self.weights.take((pad(rows), k), np.float32)
                hip.call("nc_pack_rows64", [packed, stage], [rows, k])
                hip.sync()
                return None, None, packed
            q, s = self.weights.take((rows, k), np.int8), self.weights.take((rows,), np.float32)
            at = 0
            for name in names:
                if f"{name}@int8" in weights:
                    # already quantized (the reference's quantized_weights, quantize.py:167-180,
                    # whose quantize_int8 is the same arithmetic as nc_quantize_rows_i8)
                    wq = np.ascontiguousarray(weights[f"{name}@int8"], np.int8)
                    ws = np.ascontiguousarray(weights[f"{name}@scales"], np.float32)
                    n = wq.shape[0]
                    if wq.shape[1] != k or ws.shape != (n,):
                        raise ValueError(f"{name}@int8 / @scales have shapes {wq.shape} / {ws.shape}")
                    q.view((n, k), np.int8, offset_bytes=at * k).upload(wq)
                    s.view((n,), np.float32, offset_bytes=at * 4).upload(ws)
                    at += n
                    continue
                w = np.ascontiguousarray(weights[name], np.float32)
                n = w.shape[0]
                if w.shape[1] != k:
                    raise ValueError(f"{name} has width {w.shape[1]}, expected {k}")
                view = stage.view(w.shape, np.float32)
                view.upload(w)
                hip.call("nc_quantize_rows_i8", [q.ptr + at * k, s.ptr + at * 4, view], [n, k])
                hip.sync()
                at += n
            if at != rows:
                raise ValueError(f"{names} have {at} rows, expected {rows}")
            if quantization == "int8-token":
                return q, s
            host_q = q.numpy()
            pack = pack_chains(host_q) if quantization == "int8" else pack_chains_vnni(host_q)
            packed = self.weights.take((pack.size,), np.int8)
            packed.upload(pack.reshape(-1))
            return q, s, packed

        self.layers = []
        for i in range(L):
            p = f"model.layers.{i}"
            a = f"{p}.self_attn"
            layer = {
                "g1": upload(f"{p}.input_layernorm.weight", self.weights.take((H,), np.float32)),
                "g2": upload(f"{p}.post_attention_layernorm.weight", self.weights.take((H,), np.float32)),
            }
            layer["qkv"] = quantized([f"{a}.q_proj.weight", f"{a}.k_proj.weight", f"{a}.v_proj.weight"], W, H)
            bias = self.weights.take((W,), np.float32)
            bias.upload(np.concatenate([weights[f"{a}.{n}_proj.bias"] for n in "qkv"]).astype(np.float32))
            layer["qkv_b"] = bias
            layer["o"] = quantized([f"{a}.o_proj.weight"], H, Q)
            layer["gate"] = quantized([f"{p}.mlp.gate_proj.weight"], I, H)
            layer["up"] = quantized([f"{p}.mlp.up_proj.weight"], I, H)
            layer["down"] = quantized([f"{p}.mlp.down_proj.weight"], H, I)
            self.layers.append(layer)
        self.embed = upload("model.embed_tokens.weight", self.weights.take((V, H), np.float32))
        head = self.embed
        if not c.tie_word_embeddings:
            head = DeviceArray.from_host(np.ascontiguousarray(weights["lm_head.weight"], np.float32))
        self.head = self.weights.take((vblocks, H), np.float32)
        hip.call("nc_pack_rows64", [self.head, head], [V, H])
        self.norm = upload("model.norm.weight", self.weights.take((H,), np.float32))
        self.inv_freq = self.weights.take((D // 2,), np.float32)
        self.inv_freq.upload(inverse_frequencies(D, c.rope_theta))
        self.scale = float(np.float32(D ** -0.5))
        # the fused one-token kernels exist for these widths (nc_decode.hip)
        self.fused_decode = (H, I, D) in ((896, 4864, 64), (128, 256, 32)) and Q == H \
            and quantization == "int8-token"
        hip.sync()
        del stage, head
        if self.arena.top > weight_bytes:
            raise AssertionError("the weights outgrew their region of the arena")
        self.arena.top = weight_bytes
        self.acts = self.arena
        self.x, self.qkv = self.acts.take((M, H), np.float32), self.acts.take((M, W), np.float32)
        self.ctx, self.h = self.acts.take((M, Q), np.float32), self.acts.take((M, I), np.float32)
        self.xq, self.xs = self.acts.take((M, max(I, H, Q)), np.int8), self.acts.take((M,), np.float32)
        self.normed, self.ids = self.acts.take((M, H), np.float32), self.acts.take((M,), np.int64)
        # the LM head leaves one argmax key per workgroup; the consumer reduces them
        self.slots = argmax_slots(V)
        self.best, self.logits_row = self.acts.take((self.slots,), np.uint64), self.acts.take((1, V), np.float32)
        self.argmax = self.acts.take((M,), np.int64)
        # the reference modes: gate and up apart, and the block quantizer's scales and offsets
        self.gate, self.up = self.acts.take((M, I), np.float32), self.acts.take((M, I), np.float32)
        self.xsb = self.acts.take((M, -(-max(I, H, Q) // BLOCK)), np.float32)
        self.xoff = self.acts.take((M,), np.float32)

    # -- running ---------------------------------------------------------------------

    def new_cache(self, capacity: int = 256) -> KVCache:
        if self.quantization != "int8-token" and capacity > REFERENCE_ORDER_KEYS:
            raise ValueError(f"capacity {capacity}: the reference modes' attention holds at most "
                             f"{REFERENCE_ORDER_KEYS} positions")
        return KVCache(self.config, capacity)

    def _layers(self, m: int, past: int, cache: KVCache, pos: DeviceArray | None = None) -> None:
        """The decoder layers over m new tokens at positions past .. past + m - 1.

        With ``pos`` (a device int64), the position is read on the device when
        the kernels run, so the launches can be captured once and replayed.
        """
        c = self.config
        H, I, D = c.hidden_size, c.intermediate_size, c.head_dim
        heads, kv, W = c.num_attention_heads, c.num_key_value_heads, self.width
        Q = heads * D
        eps = float_bits(c.rms_norm_eps)
        if m == 1 and self.fused_decode:
            for _, name, pointers, sizes in self.decode_layer_calls(cache, past, pos):
                hip.call(name, pointers, sizes)
            return
        if self.quantization != "int8-token":
            self._layers_reference_modes(m, past, cache, pos)
            return
        s_qkv, s_o, s_mlp, s_down = self._projection_schedules(m)
        s_attn = self.attention_schedule(m) if pos is None else 0
        for i, w in enumerate(self.layers):
            kc, vc = cache.layer(i)
            hip.call("nc_rms_norm_quant", [None, self.xq, self.xs, self.x, w["g1"]], [m, H, eps])
            q, s = w["qkv"]
            if D in (32, 64) and cache.rope is not None and _rope_schedule_ok(s_qkv, D):
                # RoPE and the cache append in the projection's epilogue (one launch); s_qkv is
                # this kernel's schedule (0, or a tile one head wide)
                hip.call("nc_matmul_i8_token_rope",
                         [self.qkv, self.xq, self.xs, q, s, w["qkv_b"], kc, vc, cache.rope, pos],
                         [m, W, H, heads, kv, D, past, cache.capacity, s_qkv])
            else:
                hip.call("nc_matmul_i8_token", [self.qkv, self.xq, self.xs, q, s, w["qkv_b"], None],
                         [m, W, H, s_qkv])
                hip.call("nc_rope_append", [self.qkv, kc, vc, self.inv_freq, pos, cache.rope],
                         [m, heads, kv, D, past, cache.capacity])
            # attention, its combine also quantizing ctx per token for the o projection
            hip.call("nc_attention", [self.ctx, self.qkv, kc, vc, pos, cache.work, self.xq, self.xs],
                     [m, heads, kv, D, past, cache.capacity, float_bits(self.scale), cache.work_bytes, s_attn])
            q, s = w["o"]
            hip.call("nc_matmul_i8_token", [self.x, self.xq, self.xs, q, s, None, self.x], [m, H, Q, s_o])
            hip.call("nc_rms_norm_quant", [None, self.xq, self.xs, self.x, w["g2"]], [m, H, eps])
            (qg, sg), (qu, su) = w["gate"], w["up"]
            hip.call("nc_matmul_i8_token_swiglu", [self.h, self.xq, self.xs, qg, sg, qu, su], [m, I, H, s_mlp])
            hip.call("nc_quantize_token_i8", [self.xq, self.xs, self.h], [m, I])
            q, s = w["down"]
            hip.call("nc_matmul_i8_token", [self.x, self.xq, self.xs, q, s, None, self.x], [m, H, I, s_down])

    def decode_layer_calls(self, cache: KVCache, past: int = 0, pos: DeviceArray | None = None) -> list[tuple]:
        """One token's pass through every layer as launches ``(label, entry point, pointers, sizes)``:
        five a layer, each projection computing its own activation prologue (nc_decode.hip) and
        attention doing RoPE and the cache append. The labels name the kernel groups a profile
        of the decode step reports: "qkv", "attention", "o", "gate/up", "down"."""
        c = self.config
        H, I, D = c.hidden_size, c.intermediate_size, c.head_dim
        heads, kv, W = c.num_attention_heads, c.num_key_value_heads, self.width
        Q = heads * D
        eps = float_bits(c.rms_norm_eps)
        s_qkv, s_o, s_mlp, s_down = self.decode_schedules()
        calls = []
        for i, w in enumerate(self.layers):
            kc, vc = cache.layer(i)
            q, s = w["qkv"]
            calls.append(("qkv", "nc_decode_projection", [self.qkv, self.x, w["g1"], q, s, w["qkv_b"]],
                          [W, H, 0, eps, s_qkv]))
            calls.append(("attention", "nc_attention_decode",
                          [self.ctx, self.qkv, kc, vc, self.inv_freq, pos, cache.rope, cache.work],
                          [heads, kv, D, past, cache.capacity, float_bits(self.scale), cache.work_bytes]))
            q, s = w["o"]
            calls.append(("o", "nc_decode_projection", [self.x, self.ctx, None, q, s], [H, Q, 1, eps, s_o]))
            (qg, sg), (qu, su) = w["gate"], w["up"]
            calls.append(("gate/up", "nc_decode_projection", [self.h, self.x, w["g2"], qg, sg, None, qu, su],
                          [I, H, 2, eps, s_mlp]))
            q, s = w["down"]
            calls.append(("down", "nc_decode_projection", [self.x, self.h, None, q, s], [H, I, 1, eps, s_down]))
        return calls

    def _layers_reference_modes(self, m: int, past: int, cache: KVCache, pos: DeviceArray | None) -> None:
        """The layers with the reference's own modes (quantize.py:127-164): float32 activations
        into matmul_i8 ("int8"), 32-wide int8 blocks into matmul_i8_vnni ("int8-vnni"), or float32
        weights ("f32"), each in the reference's k order; rms_norm and attention in the reference's
        own order too (nc_rms_norm_index_order, nc_attention_index_order: sums in index order), RoPE
        and the LM head as in "int8-token". The int8-vnni mode needs the reference's orders: its
        activations are rounded to int8 at every projection, and a last-bit difference in one of
        them can move a rounding and with it the logits by a few percent (a one-ulp change of every
        norm's gamma in the reference's own C moves its logits by 2.1% of the largest)."""
        c = self.config
        H, I, D = c.hidden_size, c.intermediate_size, c.head_dim
        heads, kv, W = c.num_attention_heads, c.num_key_value_heads, self.width
        Q = heads * D
        eps = float_bits(c.rms_norm_eps)
        for i, w in enumerate(self.layers):
            kc, vc = cache.layer(i)
            if self._fused_norm(H):                # the norm inside the projection: the same bits
                self._project_normed(w["qkv"], w["g1"], self.qkv, m, W, H, eps, bias=w["qkv_b"])
            elif self._normed_blocks(H):           # the norm inside the block quantizer: the same bits
                hip.call("nc_quantize_blocks_normed", [self.xq, self.xsb, self.xoff, self.x, w["g1"]], [m, H, eps])
                self._project(w["qkv"], None, self.qkv, m, W, H, bias=w["qkv_b"], quantized=True)
            else:
                hip.call("nc_rms_norm_index_order", [self.normed, self.x, w["g1"]], [m, H, eps])
                self._project(w["qkv"], self.normed, self.qkv, m, W, H, bias=w["qkv_b"])
            hip.call("nc_rope_append", [self.qkv, kc, vc, self.inv_freq, pos, cache.rope],
                     [m, heads, kv, D, past, cache.capacity])
            hip.call("nc_attention_index_order", [self.ctx, self.qkv, kc, vc, pos],
                     [m, heads, kv, D, past, cache.capacity, float_bits(self.scale)])
            self._project(w["o"], self.ctx, self.x, m, H, Q, residual=self.x)
            if self._normed_blocks(H):
                hip.call("nc_quantize_blocks_normed", [self.xq, self.xsb, self.xoff, self.x, w["g2"]], [m, H, eps])
                self._project(w["gate"], None, self.gate, m, I, H, quantized=True)
            else:
                hip.call("nc_rms_norm_index_order", [self.normed, self.x, w["g2"]], [m, H, eps])
                self._project(w["gate"], self.normed, self.gate, m, I, H)
            if self._silu_epilogue(H):               # SwiGLU in the up projection's epilogue: the same bits
                q, s, packed = w["up"]
                if self.quantization == "int8":
                    hip.call("nc_matmul_i8_silu", [self.h, self.normed, packed, q, s, self.gate], [m, I, H])
                else:
                    hip.call("nc_matmul_i8_vnni_silu", [self.h, self.xq, self.xsb, self.xoff, packed, q, s,
                                                        self.gate], [m, I, H, BLOCK])
            else:
                self._project(w["up"], self.normed, self.up, m, I, H, quantized=True)
                hip.call("nc_silu_mul", [self.h, self.gate, self.up], [m * I])
            self._project(w["down"], self.h, self.x, m, H, I, residual=self.x)

    def _fused_norm(self, k: int) -> bool:
        """Whether int8 mode's qkv projection takes the first norm in (nc_matmul_i8_normed, the
        model's widths; the residual stream is 256-byte aligned in the arena). Only there: its
        144 workgroups repeat the norm's chain in one round, where the gate and up projections'
        608 each would repeat it over several (measured slower)."""
        return self.quantization == "int8" and k in (896, 4864)

    def _silu_epilogue(self, k: int) -> bool:
        """Whether the reference modes' up projection applies SwiGLU in its epilogue
        (nc_matmul_i8_silu, nc_matmul_i8_vnni_silu: the model's widths)."""
        return self.quantization in ("int8", "int8-vnni") and k in (896, 4864)

    def _normed_blocks(self, k: int) -> bool:
        """Whether int8-vnni's norms run inside the block quantizer that follows them
        (nc_quantize_blocks_normed: one workgroup a row, so nothing is repeated)."""
        return self.quantization == "int8-vnni" and k <= 1024 and k % 64 == 0

    def _project_normed(self, weight, gamma, y, m: int, n: int, k: int, eps: int, bias=None) -> None:
        """rms_norm_index_order of the residual stream, then matmul_i8, in one launch."""
        q, s, packed = weight
        hip.call("nc_matmul_i8_normed", [y, self.x, packed, q, s, bias, None, gamma], [m, n, k, eps])

    def _project(self, weight, x, y, m: int, n: int, k: int, bias=None, residual=None,
                 quantized: bool = False) -> None:
        """One projection in the reference's mode; ``quantized``: int8-vnni's blocks of ``x`` are
        those the previous call left (the same input: the up projection after the gate)."""
        q, s, packed = weight
        if self.quantization == "f32":        # the reference's float32 linear: k in order, then + bias
            hip.call("nc_lm_head", [y, None, x, packed, None, bias, residual], [m, n, k, 0])
        elif self.quantization == "int8":
            hip.call("nc_matmul_i8", [y, x, packed, q, s, bias, residual], [m, n, k])
        else:
            if not quantized:
                hip.call("nc_quantize_blocks", [self.xq, self.xsb, self.xoff, x], [m, k, BLOCK])
            hip.call("nc_matmul_i8_vnni", [y, self.xq, self.xsb, self.xoff, packed, q, s, bias, residual],
                     [m, n, k, BLOCK])

    def decode_schedules(self) -> tuple[int, int, int, int]:
        """Schedules of the one-token qkv, o, gate/up and down projections (nc_decode_projection):
        0 (the library's launch shapes), or the tuner's choices, measured on first use (so call
        this before capturing a decode step, as generate does)."""
        if self.tuner is None or not self.fused_decode:
            return 0, 0, 0, 0
        if getattr(self, "_decode_schedules", None) is None:
            c = self.config
            H, I, Q = c.hidden_size, c.intermediate_size, c.num_attention_heads * c.head_dim
            if (H, I) != (896, 4864):                  # the tuned table covers the model's widths
                self._decode_schedules = (0, 0, 0, 0)
            else:
                t = self.tuner.decode_schedule
                self._decode_schedules = (t(0, self.width, H), t(1, H, Q), t(2, I, H), t(1, H, I))
        return self._decode_schedules

    def attention_schedule(self, m: int) -> int:
        """Schedule of a prompt's attention over m rows (nc_attention): 0, or the tuner's."""
        if self.tuner is None or m < 2:
            return 0
        c = self.config
        return self.tuner.attention_schedule(m, c.num_attention_heads, c.num_key_value_heads, c.head_dim)

    def _projection_schedules(self, m: int) -> tuple[int, int, int, int]:
        """Schedules of the qkv, o, gate/up and down projections over m tokens:
        0 (the library's choice), or the tuner's (measured on first use, so
        never call this first inside a graph capture)."""
        if self.tuner is None:
            return 0, 0, 0, 0
        c = self.config
        H, I, D = c.hidden_size, c.intermediate_size, c.head_dim
        Q = c.num_attention_heads * D
        t = self.tuner.schedule
        if D in (32, 64) and self.quantization == "int8-token" and m > 1:
            # the qkv projection runs with RoPE and the cache append in its epilogue: tune that kernel
            qkv = self.tuner.rope_schedule(m, self.width, H, c.num_attention_heads, c.num_key_value_heads, D)
        else:
            qkv = t("matmul_i8_token", m, self.width, H)
        return (qkv, t("matmul_i8_token", m, H, Q), t("matmul_i8_token_swiglu", m, I, H), t("matmul_i8_token", m, H, I))

    def forward(self, token_ids: Sequence[int] | np.ndarray, cache: KVCache | None = None,
                last_only: bool = False) -> np.ndarray:
        """Logits for ``token_ids``, the tokens not already in ``cache`` (models/qwen2.py:316-345)."""
        ids = np.asarray(token_ids, dtype=np.int64)
        if ids.ndim != 1 or ids.size == 0:
            raise ValueError(f"expected a non-empty 1-D sequence of token IDs, got {ids.shape}")
        m = int(ids.size)
        if m > self.max_tokens:
            raise ValueError(f"{m} tokens in one forward; this model was made for at most {self.max_tokens}")
        held = cache is not None
        if cache is None:
            cache = self.new_cache(m)
        past = cache.length
        if past + m > cache.capacity:
            raise ValueError(f"the cache holds {cache.capacity} tokens; {past} + {m} do not fit")
        c = self.config
        H, V = c.hidden_size, c.vocab_size
        if m == 1 and held:
            # one token into a caller's cache: the step replayed from a graph captured for this
            # cache, the position read on the device (the same kernels, the same bits as
            # launching them one by one)
            self.ids.view((1,)).upload(ids)
            cache.position.upload(np.array([past], np.int64))
            self._step_graph(cache).launch()
            hip.sync()
            cache.length = past + 1
            return self.logits_row.numpy()[:1]
        self.ids.view((m,)).upload(ids)
        hip.call("nc_embed", [self.x, self.embed, self.ids], [m, H, V])
        self._layers(m, past, cache)
        rows = 1 if last_only else m
        first = m - rows
        x_rows = self.x.ptr + first * H * 4
        self._final_norm(x_rows, rows)
        logits = self.logits_row if rows == 1 else DeviceArray((rows, V), np.float32)
        hip.call("nc_lm_head", [logits, None, self.normed, self.head], [rows, V, H])
        hip.sync()
        cache.length = past + m
        return logits.numpy()[:rows]

    def _step_graph(self, cache: KVCache):
        """A one-token forward for ``cache`` captured as a HIP graph: the embedding of ``ids``, every
        layer at the position ``cache.position`` holds, the final rms_norm and the LM head's logits
        row. Made on a cache's first one-token call and kept, with a reference to the cache, for
        the latest cache only (a caller's sequence of steps replays it; switching between caches
        captures again); any tuning happens before the capture."""
        held = getattr(self, "_held_step", None)
        if held is not None and held[0] is cache:
            return held[1]
        c = self.config
        H, V = c.hidden_size, c.vocab_size
        self._projection_schedules(1)
        self.decode_schedules()
        hip.sync()

        def step() -> None:
            hip.call("nc_embed", [self.x, self.embed, self.ids], [1, H, V])
            self._layers(1, 0, cache, pos=cache.position)
            self._final_norm(self.x.ptr, 1)
            hip.call("nc_lm_head", [self.logits_row, None, self.normed, self.head], [1, V, H])

        graph = hip.Graph.capture(step)
        self._held_step = (cache, graph)
        return graph

    def next_token(self, token_ids, cache: KVCache) -> int:
        """Greedy's step on the device: forward the new tokens, return the argmax of the last row."""
        ids = np.asarray(token_ids, dtype=np.int64)
        m = int(ids.size)
        past = cache.length
        if m == 0 or m > self.max_tokens or past + m > cache.capacity:
            raise ValueError("token count outside the model's or the cache's limits")
        c = self.config
        H, V = c.hidden_size, c.vocab_size
        self.ids.view((m,)).upload(ids)
        hip.call("nc_embed", [self.x, self.embed, self.ids], [m, H, V])
        self._layers(m, past, cache)
        self._final_norm(self.x.ptr + (m - 1) * H * 4, 1)
        hip.call("nc_lm_head", [None, self.best, self.normed, self.head], [1, V, H, 0, 1])
        hip.call("nc_argmax_index", [self.argmax, self.best], [1, self.slots])
        token = int(self.argmax.view((1,)).numpy()[0])      # waits for the stream; a failed copy raises
        hip.sync()                                             # a kernel's failure code raises KernelError
        cache.length = past + m
        return token


    # -- greedy decoding on the device -------------------------------------------------

    def _final_norm(self, rows_ptr: int, rows: int) -> None:
        """The final rms_norm of ``rows`` rows into ``normed``: the reference's index order in its
        own modes, the row kernels' order in "int8-token"."""
        c = self.config
        eps = float_bits(c.rms_norm_eps)
        if self.quantization == "int8-token":
            hip.call("nc_rms_norm_quant", [self.normed, self.xq, self.xs, rows_ptr, self.norm],
                     [rows, c.hidden_size, eps])
        else:
            hip.call("nc_rms_norm_index_order", [self.normed, rows_ptr, self.norm], [rows, c.hidden_size, eps])

    def _head_argmax(self, row_ptr: int) -> None:
        """Final rms_norm of one row and the LM head (one kernel in "int8-token"; the norm in the
        reference's order first in its own modes), its argmax keys (one per workgroup) into ``best``."""
        c = self.config
        H, V = c.hidden_size, c.vocab_size
        if self.quantization != "int8-token":
            self._final_norm(row_ptr, 1)
            hip.call("nc_lm_head", [None, self.best, self.normed, self.head], [1, V, H, 0, 1])
            return
        hip.call("nc_lm_head", [None, self.best, row_ptr, self.head, self.norm],
                 [1, V, H, float_bits(c.rms_norm_eps), 1])

    def generate(self, prompt_ids: Sequence[int], max_new_tokens: int, timer=None, graph: bool = True) -> list[int]:
        """Greedy decoding with the whole loop on the device; the same tokens as :func:`greedy`.

        The prompt runs as one forward; each following token is one replay of
        a HIP graph holding a whole decode step (embedding, every layer, the
        LM head, the argmax and the bookkeeping that feeds the token back),
        with the position read on the device. ``timer``, if given, is called
        as ``timer(i)`` before replay ``i`` (0 .. max_new_tokens - 2) and as
        ``timer(max_new_tokens - 1)`` after the last, from the host as the
        replays are enqueued (a caller records events on the library stream
        at the indices it wants).
        """
        prompt = np.asarray(prompt_ids, dtype=np.int64)
        m = int(prompt.size)
        if m == 0 or max_new_tokens <= 0:
            raise ValueError("need a non-empty prompt and at least one new token")
        if m > self.max_tokens:
            raise ValueError(f"a {m}-token prompt; this model was made for at most {self.max_tokens}")
        c = self.config
        H, V = c.hidden_size, c.vocab_size
        capacity = m + max_new_tokens
        cache = self.new_cache(capacity)
        tokens, pos = cache.tokens, cache.position
        one_id = self.acts.base.view((1,), np.int64, offset_bytes=self.ids.ptr - self.acts.base.ptr)

        self.ids.view((m,)).upload(prompt)
        hip.call("nc_embed", [self.x, self.embed, self.ids], [m, H, V])
        self._layers(m, 0, cache)
        self._head_argmax(self.x.ptr + (m - 1) * H * 4)
        pos.upload(np.array([m - 1], np.int64))
        # the advance also gathers the next token's embedding row into x
        advance = ("nc_decode_advance", [one_id, tokens, self.best, pos, self.x, self.embed],
                   [capacity, H, V, self.slots])
        hip.call(*advance)

        def step() -> None:
            self._layers(1, 0, cache, pos=pos)
            self._head_argmax(self.x.ptr)
            hip.call(*advance)

        if not self.fused_decode:
            self._projection_schedules(1)          # any tuning happens now, not under capture
        self.decode_schedules()
        hip.sync()
        replay = hip.Graph.capture(step).launch if graph else step
        for i in range(max_new_tokens - 1):
            if timer:
                timer(i)
            replay()
        if timer:
            timer(max_new_tokens - 1)
        hip.sync()
        cache.length = capacity - 1
        return [int(t) for t in tokens.numpy()[m:capacity]]


def greedy(model: Qwen2, prompt_ids: Sequence[int], max_new_tokens: int, use_cache: bool = True) -> list[int]:
    """Argmax decoding (models/qwen2.py:348-368)."""
    if not prompt_ids:
        raise ValueError("cannot generate from an empty prompt")
    ids = list(prompt_ids)
    cache = model.new_cache(len(ids) + max_new_tokens) if use_cache else None
    pending = ids
    generated: list[int] = []
    for _ in range(max_new_tokens):
        if use_cache:
            token = model.next_token(pending, cache)
        else:
            token = int(np.argmax(model.forward(pending, last_only=True)[0]))
        generated.append(token)
        ids.append(token)
        pending = [token] if use_cache else ids
    return generated
