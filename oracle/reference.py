"""CPU restatement of the reference's int8 path, in NumPy. TEST INFRASTRUCTURE ONLY.

This module is the checker, never the thing measured or shipped: only
``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg
import it. The product (``nanocompile_amd``) never does, and has no CPU
fallback.

Every function follows a reference function, cited by file:line in
/root/reference (SpookyJumpyBeans/nanocompile). Float32 arithmetic is done one
IEEE operation at a time on float32 arrays (NumPy's elementwise float32 add,
multiply, divide and sqrt are correctly rounded), and sums that have an order
are written as loops in that order, never ``np.sum`` (which is pairwise).

How each function is pinned (tests/test_oracle.py and tests/golden/):
  quantize_int8        the reference's own special rows (test_int8.py:70-78)
                       and golden vectors G1 made by the reference
  round_half_away      the 16 known values of test_int8.py:82-88
  quantize_token       closed form: the per-token case of quantize.py:102-124,
                       checked against quantize_blocks with block = K and
                       against invariants (|xq| <= 127, max -> +-127)
  quantize_blocks      golden vectors G3 (the reference's graph ops)
  matmul_i8_token_acc  brute force in Python integers on small shapes
  matmul_i8_token      its epilogue checked op by op in float64-exact form
  rms_norm_reference   golden vectors G4 from the reference's row kernel
  rms_norm_gpu_order   the same function as rms_norm_reference up to the
                       order of one sum (bounded), and exact on rows whose
                       squares sum exactly (powers of two)
  attention_index_order  float64 attention (within rounding), golden G4's
                       softmax with the mask (the reference's row kernel) for
                       its softmax step, a planted dropped max failing the
                       first; end to end, golden G6's int8-vnni tokens, which
                       move with any last-bit difference in the activations
"""

from __future__ import annotations

import numpy as np

INT8_MAX = 127
F32 = np.float32


# -- rounding and quantizers ---------------------------------------------------


def round_half_away(x: np.ndarray) -> np.ndarray:
    """C's roundf on float32: interpreter.py:192-201 (exact in float64)."""
    x = np.asarray(x, dtype=F32)
    wide = x.astype(np.float64)
    rounded = np.copysign(np.floor(np.abs(wide) + 0.5), wide)
    return np.where(np.abs(wide) < 2.0**23, rounded, wide).astype(F32)


def quantize_int8(weights: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Per-row int8 weights and f32 scales: quantize.py:55-70, operation for operation.

    The rounding is float32 ``sign(s) * floor(|s| + 0.5)``: 0.49999997 rounds
    to 1 here (|s| + 0.5 rounds up in float32), where roundf gives 0.
    """
    w = np.asarray(weights, dtype=F32)
    if w.ndim != 2:
        raise ValueError(f"expected a 2-D weight matrix, got shape {w.shape}")
    scales = (np.max(np.abs(w), axis=1) / F32(INT8_MAX)).astype(F32)
    scales[scales == 0] = F32(1.0)
    scaled = (w / scales[:, None]).astype(F32)
    rounded = (np.sign(scaled) * np.floor(np.abs(scaled) + F32(0.5))).astype(F32)
    values = np.clip(rounded, -INT8_MAX, INT8_MAX).astype(np.int8)
    return values, scales.astype(F32)


def clamp_int8(rounded: np.ndarray) -> np.ndarray:
    """The activation quantizer's clamp as two selects (quantize.py:116-118):
    ``where(r <= 127, r, 127)`` then ``where(-127 <= c, c, -127)``, so a NaN
    (a row whose scale is NaN or infinite) becomes 127, not numpy's cast of NaN."""
    clamped = np.where(rounded <= F32(INT8_MAX), rounded, F32(INT8_MAX))
    clamped = np.where(F32(-INT8_MAX) <= clamped, clamped, F32(-INT8_MAX))
    return clamped.astype(np.int8)


def quantize_token(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Per-token int8 activations: quantize.py:102-124 with one block spanning the row.

    ``mag = max|x|``; ``scale = 1 if mag <= 0 else mag / 127``;
    ``xq = clamp(round(x / scale), -127, 127)`` with round half away from zero.
    """
    x = np.asarray(x, dtype=F32)
    magnitude = np.max(np.where(F32(0) <= x, x, -x), axis=-1) if x.shape[-1] else np.zeros(x.shape[:-1], F32)
    scale = np.where(magnitude <= 0, F32(1.0), (magnitude / F32(INT8_MAX)).astype(F32)).astype(F32)
    rounded = round_half_away((x / scale[..., None]).astype(F32))
    return clamp_int8(rounded), scale


def quantize_blocks(x: np.ndarray, block: int = 32) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Block activation quantization for matmul_i8_vnni: quantize.py:102-124.

    Returns ``(xq i8[..., K], xs f32[..., K / block], offset f32[..., 1])`` with
    ``offset = 128 * sum_b f32(sum(xq_b)) * xs_b`` summed over blocks in order.
    """
    x = np.asarray(x, dtype=F32)
    k = x.shape[-1]
    if k % block:
        raise ValueError(f"width {k} is not a whole number of blocks of {block}")
    lead, blocks = x.shape[:-1], k // block
    groups = x.reshape(lead + (blocks, block))
    magnitude = np.max(np.where(F32(0) <= groups, groups, -groups), axis=-1)
    scale = np.where(magnitude <= 0, F32(1.0), (magnitude / F32(INT8_MAX)).astype(F32)).astype(F32)
    with np.errstate(invalid="ignore"):            # a NaN block's scale is NaN: its values, as C's
        rounded = round_half_away((groups / scale[..., None]).astype(F32))
    values = clamp_int8(rounded)
    block_sums = values.astype(np.int32).sum(-1).astype(F32)
    terms = (block_sums * scale).astype(F32)
    total = np.zeros(lead, F32)
    for b in range(blocks):                         # reduce_sum over the blocks, in order
        total = (total + terms[..., b]).astype(F32)
    offset = (total * F32(128.0)).astype(F32)[..., None]
    return values.reshape(lead + (k,)), scale, offset


# -- the per-token int8 projection (matmul_i8_token) ---------------------------


def matmul_i8_token_acc(xq: np.ndarray, q: np.ndarray) -> np.ndarray:
    """``xq @ q.T`` exactly (int64), as int32: every order gives these integers."""
    acc = np.asarray(xq).astype(np.int64) @ np.asarray(q).astype(np.int64).T
    if np.abs(acc).max(initial=0) >= 2**31:
        raise OverflowError("an int8 dot product does not fit int32")
    return acc.astype(np.int32)


def matmul_i8_token(xq, xs, q, scales, bias=None, residual=None) -> np.ndarray:
    """The frozen epilogue: ``(f32(acc) * xs[m]) * scales[n]``, then ``+ bias``, then ``residual +``."""
    acc = matmul_i8_token_acc(xq, q)
    y = (acc.astype(F32) * np.asarray(xs, F32)[:, None]).astype(F32)
    y = (y * np.asarray(scales, F32)[None, :]).astype(F32)
    if bias is not None:
        y = (y + np.asarray(bias, F32)[None, :]).astype(F32)
    if residual is not None:
        y = (np.asarray(residual, F32) + y).astype(F32)
    return y


# -- rms_norm ------------------------------------------------------------------


def _rms_finish(x: np.ndarray, ss: np.ndarray, gamma: np.ndarray, eps: float) -> np.ndarray:
    """``(x * (1 / sqrt(ss / K + eps))) * gamma``: nn.py:34-38 after the sum."""
    k = x.shape[-1]
    ms = (ss / F32(k)).astype(F32)
    rcp = (F32(1.0) / np.sqrt((ms + F32(eps)).astype(F32))).astype(F32)
    return ((x * rcp[:, None]).astype(F32) * np.asarray(gamma, F32)[None, :]).astype(F32)


def rms_norm_reference(x: np.ndarray, gamma: np.ndarray, eps: float) -> np.ndarray:
    """The reference's row kernel: the sum of squares in index order (fusion.py:631-650)."""
    x = np.asarray(x, dtype=F32)
    ss = np.zeros(x.shape[0], F32)
    for r in range(x.shape[1]):
        ss = (ss + (x[:, r] * x[:, r]).astype(F32)).astype(F32)
    return _rms_finish(x, ss, gamma, eps)


THREADS = 256


def gpu_row_sum(values: np.ndarray) -> np.ndarray:
    """The order of the GPU row kernels' float sum over each row of ``values``.

    Thread t adds elements t, t + 256, ... in order from 0; each wave of 64
    threads sums by the xor butterfly (offsets 32, 16, 8, 4, 2, 1); the four
    wave sums combine as (w0 + w1) + (w2 + w3). Padding with +0.0 adds
    nothing: every partial sum here is a sum of squares, never -0.0.
    """
    values = np.asarray(values, dtype=F32)
    m, k = values.shape
    per = max(1, -(-k // THREADS))
    padded = np.zeros((m, per * THREADS), F32)
    padded[:, :k] = values
    s = np.zeros((m, THREADS), F32)
    for i in range(per):
        s = (s + padded[:, i * THREADS:(i + 1) * THREADS]).astype(F32)
    s = s.reshape(m, 4, 64)
    lanes = np.arange(64)
    for off in (32, 16, 8, 4, 2, 1):
        s = (s + s[:, :, lanes ^ off]).astype(F32)
    w = s[:, :, 0]
    return ((w[:, 0] + w[:, 1]).astype(F32) + (w[:, 2] + w[:, 3]).astype(F32)).astype(F32)


def rms_norm_gpu_order(x: np.ndarray, gamma: np.ndarray, eps: float) -> np.ndarray:
    """rms_norm with the sum of squares in the GPU row kernels' order."""
    x = np.asarray(x, dtype=F32)
    ss = gpu_row_sum((x * x).astype(F32))
    return _rms_finish(x, ss, gamma, eps)


def rms_norm_quant_gpu_order(x, gamma, eps):
    """rms_norm (GPU order), then per-token int8: ``(normed, xq, xs)``."""
    normed = rms_norm_gpu_order(x, gamma, eps)
    xq, xs = quantize_token(normed)
    return normed, xq, xs


# -- the reference's attention in its own order ----------------------------------


def softmax_index_order(z: np.ndarray, exp) -> np.ndarray:
    """The reference's softmax over the last axis (nn.py:57-66): shifted = exp(z - max z); the
    sum of shifted in index order from 0; shifted / sum. ``exp`` is the float32 exponential to
    use (the reference's C calls the C library's expf, codegen_c.py:58)."""
    z = np.asarray(z, F32)
    m = z.max(axis=-1, keepdims=True)
    shifted = np.asarray(exp((z - m).astype(F32)), F32).reshape(z.shape)
    total = np.zeros(z.shape[:-1] + (1,), F32)
    for t in range(z.shape[-1]):
        total = (total + shifted[..., t:t + 1]).astype(F32)
    return (shifted / total).astype(F32)


def attention_index_order(q: np.ndarray, kcache: np.ndarray, vcache: np.ndarray, past: int, scale: float,
                          exp) -> np.ndarray:
    """The reference's grouped-query attention for M new rows (models/qwen2.py:143-147 with
    nn.py:57-66, 109-135), each sum in its order: ``q`` [M, heads, D] (rotated), ``kcache`` /
    ``vcache`` [kv, >= past + M, D] holding the rows' own keys and values at past .. past + M - 1.
    Scores: for each position a dot product over d in order (one multiply and one add a step,
    from 0), times scale, plus the mask (0 where visible). Row i sees positions 0 .. past + i;
    the masked rest would add exp(-inf) = 0 to the softmax's sum and 0 * v to each context sum,
    changing no float, so only the visible ones are summed. Context: the sum over positions in
    order of p_t * v_t. Returns [M, heads, D]."""
    q = np.asarray(q, F32)
    m_rows, heads, d = q.shape
    kv = kcache.shape[0]
    group = heads // kv
    out = np.zeros((m_rows, heads, d), F32)
    for i in range(m_rows):
        t_end = past + i + 1
        k = np.repeat(np.asarray(kcache[:, :t_end], F32), group, axis=0)        # [heads, T, D]
        v = np.repeat(np.asarray(vcache[:, :t_end], F32), group, axis=0)
        acc = np.zeros((heads, t_end), F32)
        for j in range(d):
            acc = (acc + (q[i, :, j:j + 1] * k[:, :, j]).astype(F32)).astype(F32)
        z = ((acc * F32(scale)).astype(F32) + F32(0.0)).astype(F32)
        p = softmax_index_order(z, exp)
        ctx = np.zeros((heads, d), F32)
        for t in range(t_end):
            ctx = (ctx + (p[:, t:t + 1] * v[:, t, :]).astype(F32)).astype(F32)
        out[i] = ctx
    return out
