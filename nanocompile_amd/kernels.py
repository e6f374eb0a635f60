"""The hot path's operators on device arrays, with the reference's typing contracts.

Each function checks its operands the way the reference's IR checks a node's
(ir.py:381-439: one f32 scale per i8 weight row, activations of the weights'
width) and raises :class:`ShapeError` with the same kind of message, then
enqueues one kernel of the HIP library. Results are :class:`DeviceArray`\\ s;
nothing is copied to the host unless the caller asks.
"""

from __future__ import annotations

import numpy as np

from nanocompile_amd import hip
from nanocompile_amd.hip import DeviceArray

F32, I8, I32 = np.dtype(np.float32), np.dtype(np.int8), np.dtype(np.int32)


class ShapeError(ValueError):
    """Operands that do not fit the primitive (the reference's ir.ShapeError)."""


SHORT = {F32: "f32", I8: "i8", I32: "i32", np.dtype(np.int64): "i64"}


def _device(x, dtype=None) -> DeviceArray:
    """``x`` on the device (uploaded if it is a host array), checked to be ``dtype``."""
    have = x.dtype if isinstance(x, DeviceArray) else np.asarray(x).dtype
    if dtype is not None and have != np.dtype(dtype):
        want = SHORT.get(np.dtype(dtype), str(dtype))
        raise ShapeError(f"operand must be {want}, got {SHORT.get(have, str(have))}")
    return x if isinstance(x, DeviceArray) else DeviceArray.from_host(np.asarray(x))


def float_bits(value: float) -> int:
    return int(np.array(value, dtype=np.float32).view(np.uint32))


# The most keys (cached plus new) one attention launch takes: its combine step
# keeps one float per key of a row in LDS (nc_attention.hip kMaxKeys).
MAX_KEYS = 16384


def attention_workspace_bytes(heads: int, head_dim: int, rows: int, keys: int) -> int:
    """Bytes of the chunk results nc_attention / nc_attention_decode keep for ``rows``
    query rows over ``keys`` keys: (m, l, o[head_dim]) per head, row and 64-key chunk."""
    return heads * rows * -(-keys // 64) * (head_dim + 2) * 4


def argmax_slots(vocab: int) -> int:
    """Argmax keys per row that nc_lm_head leaves with s[4] = 1: one per workgroup of 64 rows."""
    return -(-vocab // 64)


def _int8_weight(op: str, q: DeviceArray, scales: DeviceArray, k: int) -> int:
    """Check ``q: i8[N, K]`` and ``scales: f32[N]`` against width ``k``; return N (ir.py:381-389)."""
    if q.dtype != I8 or len(q.shape) != 2:
        raise ShapeError(f"{op}: weights must be i8[N, K], got {q.dtype}{list(q.shape)}")
    if scales.dtype != F32 or len(scales.shape) != 1 or scales.shape[0] != q.shape[0]:
        raise ShapeError(f"{op}: expected one f32 scale per row of i8{list(q.shape)}, "
                         f"got {scales.dtype}{list(scales.shape)}")
    if q.shape[1] != k:
        raise ShapeError(f"{op}: activations have width {k}, weights i8{list(q.shape)} expect {q.shape[1]}")
    return q.shape[0]


def quantize_int8(w) -> tuple[DeviceArray, DeviceArray]:
    """Per-row symmetric int8 of an ``[N, K]`` f32 matrix: (values, scales) (quantize.py:55-70)."""
    w = _device(w, F32)
    if len(w.shape) != 2:
        raise ValueError(f"expected a 2-D weight matrix, got shape {w.shape}")
    n, k = w.shape
    q, scales = DeviceArray((n, k), I8), DeviceArray((n,), F32)
    if n and k:
        hip.call("nc_quantize_rows_i8", [q, scales, w], [n, k])
    return q, scales


def quantize_token(x) -> tuple[DeviceArray, DeviceArray]:
    """``x: f32[M, K]`` to ``(xq i8[M, K], xs f32[M])``: one scale per token."""
    x = _device(x, F32)
    if len(x.shape) != 2:
        raise ShapeError(f"quantize_token: activations must be f32[M, K], got {list(x.shape)}")
    m, k = x.shape
    xq, xs = DeviceArray((m, k), I8), DeviceArray((m,), F32)
    if m and k:
        hip.call("nc_quantize_token_i8", [xq, xs, x], [m, k])
    return xq, xs


def rms_norm_quant(x, gamma, eps: float, normed: bool = True):
    """rms_norm then per-token int8, one kernel: ``(normed | None, xq, xs)``."""
    x, gamma = _device(x, F32), _device(gamma, F32)
    if len(x.shape) != 2 or gamma.shape != (x.shape[1],):
        raise ShapeError(f"rms_norm_quant: x f32[M, K] and gamma f32[K], got {list(x.shape)}, {list(gamma.shape)}")
    m, k = x.shape
    out = DeviceArray((m, k), F32) if normed else None
    xq, xs = DeviceArray((m, k), I8), DeviceArray((m,), F32)
    if m:
        hip.call("nc_rms_norm_quant", [out, xq, xs, x, gamma], [m, k, float_bits(eps)])
    return out, xq, xs


def matmul_i8_token(xq, xs, q, scales, bias=None, residual=None, schedule: int = 0) -> DeviceArray:
    """``(f32(xq @ q.T) * xs[:, None]) * scales (+ bias) (+ residual)``, accumulated exactly in int32."""
    xq, xs, q, scales = _device(xq, I8), _device(xs, F32), _device(q, I8), _device(scales, F32)
    if len(xq.shape) != 2:
        raise ShapeError(f"matmul_i8_token: activations must be i8[M, K], got {list(xq.shape)}")
    m, k = xq.shape
    if xs.shape != (m,):
        raise ShapeError(f"matmul_i8_token: expected f32[{m}] token scales, got {list(xs.shape)}")
    n = _int8_weight("matmul_i8_token", q, scales, k)
    if bias is not None:
        bias = _device(bias, F32)
        if bias.shape != (n,):
            raise ShapeError(f"matmul_i8_token: bias must be f32[{n}]")
    if residual is not None:
        residual = _device(residual, F32)
        if residual.shape != (m, n):
            raise ShapeError(f"matmul_i8_token: residual must be f32[{m}, {n}]")
    y = DeviceArray((m, n), F32)
    hip.call("nc_matmul_i8_token", [y, xq, xs, q, scales, bias, residual], [m, n, k, schedule])
    return y


GEMV_SCHEDULES = range(1, 8)      # lanes per row x waves; 7 is the default GEMV
GEMM_SCHEDULES = range(16, 25)    # the MFMA GEMM's tiles; K a multiple of 16


def matmul_i8_token_swiglu(xq, xs, qg, sg, qu, su, schedule: int = 0) -> DeviceArray:
    """``silu(gate) * up`` with gate and up each ``(f32(xq @ q.T) * xs) * scales``, one kernel."""
    xq, xs = _device(xq, I8), _device(xs, F32)
    if len(xq.shape) != 2 or xs.shape != (xq.shape[0],):
        raise ShapeError(f"matmul_i8_token_swiglu: activations i8[M, K] and f32[M], got {list(xq.shape)}")
    m, k = xq.shape
    qg, sg, qu, su = _device(qg, I8), _device(sg, F32), _device(qu, I8), _device(su, F32)
    n = _int8_weight("matmul_i8_token_swiglu", qg, sg, k)
    if _int8_weight("matmul_i8_token_swiglu", qu, su, k) != n:
        raise ShapeError("matmul_i8_token_swiglu: gate and up must have the same rows")
    h = DeviceArray((m, n), F32)
    hip.call("nc_matmul_i8_token_swiglu", [h, xq, xs, qg, sg, qu, su], [m, n, k, schedule])
    return h


def matmul_i8_token_acc(xq, q, schedule: int = 0) -> DeviceArray:
    """The int32 accumulators ``xq @ q.T`` alone, for checking them bit for bit."""
    xq, q = _device(xq, I8), _device(q, I8)
    if len(xq.shape) != 2 or len(q.shape) != 2 or xq.shape[1] != q.shape[1]:
        raise ShapeError(f"matmul_i8_token_acc: i8[M, K] @ i8[N, K].T, got {list(xq.shape)}, {list(q.shape)}")
    m, k = xq.shape
    acc = DeviceArray((m, q.shape[0]), I32)
    hip.call("nc_matmul_i8_token_acc", [acc, xq, q], [m, q.shape[0], k, schedule])
    return acc


def matmul_i8_token_stacked(xq, xs, q, scales, out: DeviceArray | None = None, schedule: int = 0) -> DeviceArray:
    """``B`` independent projections in one launch: ``xq i8[B,M,K]``, ``q i8[B,N,K]`` -> ``f32[B,M,N]``."""
    xq, xs, q, scales = _device(xq, I8), _device(xs, F32), _device(q, I8), _device(scales, F32)
    if len(xq.shape) != 3 or len(q.shape) != 3 or xq.shape[0] != q.shape[0] or xq.shape[2] != q.shape[2]:
        raise ShapeError(f"matmul_i8_token_stacked: i8[B,M,K] and i8[B,N,K], got {list(xq.shape)}, {list(q.shape)}")
    b, m, k = xq.shape
    n = q.shape[1]
    if xs.shape != (b, m) or scales.shape != (b, n):
        raise ShapeError("matmul_i8_token_stacked: scales must be f32[B,M] and f32[B,N]")
    if out is None:
        out = DeviceArray((b, m, n), F32)
    hip.call("nc_matmul_i8_token_stacked", [out, xq, xs, q, scales], [b, m, n, k, schedule])
    return out


# -- the reference's two int8 modes (matmul_i8, matmul_i8_vnni) ----------------------


def pack_chains(q: np.ndarray) -> np.ndarray:
    """matmul_i8's weight layout: per row, per group of 4 whole 32-blocks, lane l's 16 bytes
    are [block][c] = w[32*k0 + 8c + l] (zeros past the last block)."""
    q = np.ascontiguousarray(q, np.int8)
    n, k = q.shape
    blocks = k // 32
    quads = -(-blocks // 4)
    wide = np.zeros((n, quads * 4, 4, 8), np.int8)                      # (n, k0, c, l)
    wide[:, :blocks] = q[:, :blocks * 32].reshape(n, blocks, 4, 8)
    return np.ascontiguousarray(wide.reshape(n, quads, 4, 4, 8).transpose(0, 1, 4, 2, 3))   # (n, j, l, kk, c)


def pack_chains_vnni(q: np.ndarray) -> np.ndarray:
    """matmul_i8_vnni's weight layout: per row, per 128-block, lane l's 16 bytes are the
    four dwords w[128*k0 + 32c + 4l .. + 3], c = 0..3."""
    q = np.ascontiguousarray(q, np.int8)
    n, k = q.shape
    strides = k // 128
    wide = q[:, :strides * 128].reshape(n, strides, 4, 8, 4)             # (n, k0, c, l, j)
    return np.ascontiguousarray(wide.transpose(0, 1, 3, 2, 4))            # (n, k0, l, c, j)


def _epilogue_operands(op, n, m, bias, residual):
    if bias is not None:
        bias = _device(bias, F32)
        if bias.shape != (n,):
            raise ShapeError(f"{op}: bias must be f32[{n}]")
    if residual is not None:
        residual = _device(residual, F32)
        if residual.shape != (m, n):
            raise ShapeError(f"{op}: residual must be f32[{m}, {n}]")
    return bias, residual


def matmul_i8(x, q, scales, packed=None, bias=None, residual=None) -> DeviceArray:
    """The reference's matmul_i8 (ir.py:392-406): float activations, per-row int8 weights,
    the 32-chain FMA order of lower.py:294-356, bit for bit."""
    x, scales = _device(x, F32), _device(scales, F32)
    if len(x.shape) != 2:
        raise ShapeError(f"matmul_i8: activations must be f32[M, K], got {list(x.shape)}")
    m, k = x.shape
    host_q = q.numpy() if isinstance(q, DeviceArray) else np.asarray(q)
    q = _device(q, I8)
    n = _int8_weight("matmul_i8", q, scales, k)
    packed = _device(pack_chains(host_q) if packed is None else packed, I8)
    bias, residual = _epilogue_operands("matmul_i8", n, m, bias, residual)
    y = DeviceArray((m, n), F32)
    hip.call("nc_matmul_i8", [y, x, packed, q, scales, bias, residual], [m, n, k])
    return y


def quantize_blocks(x, block: int = 32) -> tuple[DeviceArray, DeviceArray, DeviceArray]:
    """Block activation quantization (quantize.py:102-124): (xq i8[M,K], xs f32[M,K/block], offset f32[M])."""
    x = _device(x, F32)
    if len(x.shape) != 2:
        raise ShapeError(f"quantize_blocks: activations must be f32[M, K], got {list(x.shape)}")
    m, k = x.shape
    if k % block:
        raise ValueError(f"width {k} is not a whole number of blocks of {block}")
    xq, xs, offset = DeviceArray((m, k), I8), DeviceArray((m, k // block), F32), DeviceArray((m,), F32)
    if m:
        hip.call("nc_quantize_blocks", [xq, xs, offset, x], [m, k, block])
    return xq, xs, offset


def matmul_i8_vnni(xq, xs, offset, q, scales, block: int = 32, packed=None, bias=None,
                   residual=None) -> DeviceArray:
    """The reference's matmul_i8_vnni (ir.py:409-439) in the order of lower.py:359-397, bit for bit."""
    if not (isinstance(block, int) and block >= 32 and block & (block - 1) == 0):
        raise ShapeError(f"matmul_i8_vnni: block must be a power of two >= 32, got {block!r}")
    xq, xs, offset, scales = _device(xq, I8), _device(xs, F32), _device(offset, F32), _device(scales, F32)
    if len(xq.shape) != 2:
        raise ShapeError(f"matmul_i8_vnni: activations must be i8[M, K], got {list(xq.shape)}")
    m, k = xq.shape
    if k % block:
        raise ShapeError(f"matmul_i8_vnni: width {k} is not a whole number of blocks of {block}")
    if xs.shape != (m, k // block) or offset.shape not in ((m,), (m, 1)):
        raise ShapeError("matmul_i8_vnni: expected f32[M, K/block] scales and f32[M, 1] offsets")
    host_q = q.numpy() if isinstance(q, DeviceArray) else np.asarray(q)
    q = _device(q, I8)
    n = _int8_weight("matmul_i8_vnni", q, scales, k)
    packed = _device(pack_chains_vnni(host_q) if packed is None else packed, I8)
    bias, residual = _epilogue_operands("matmul_i8_vnni", n, m, bias, residual)
    y = DeviceArray((m, n), F32)
    hip.call("nc_matmul_i8_vnni", [y, xq, xs, offset, packed, q, scales, bias, residual], [m, n, k, block])
    return y
