"""ctypes front end of the host C oracle/baseline (``nc_host.c``). TEST INFRASTRUCTURE ONLY."""

from __future__ import annotations

import ctypes

import numpy as np

from oracle.build import LIBRARY

ISA_NAMES = {0: "scalar", 1: "avx2", 2: "avx-vnni", 3: "avx512-vnni"}
_LIB = None
_P = ctypes.c_void_p
_I = ctypes.c_int64


def load() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        if not LIBRARY.exists():
            raise RuntimeError(f"{LIBRARY} is not built; run python -m oracle.build")
        lib = ctypes.CDLL(str(LIBRARY))
        lib.nc_host_set_threads.argtypes, lib.nc_host_set_threads.restype = [ctypes.c_int], ctypes.c_int
        lib.nc_host_threads.restype = ctypes.c_int
        lib.nc_host_isa.restype = ctypes.c_int
        lib.nc_host_limit_isa.argtypes, lib.nc_host_limit_isa.restype = [ctypes.c_int], ctypes.c_int
        lib.nc_host_matmul_i8_token.argtypes = [_P] * 7 + [_I] * 3
        lib.nc_host_matmul_i8_token_acc.argtypes = [_P] * 3 + [_I] * 3
        lib.nc_host_time_matmul_i8_token.argtypes = [_P] * 5 + [_I] * 5
        lib.nc_host_time_matmul_i8_token.restype = ctypes.c_double
        lib.nc_host_read_gbps.argtypes = [_P, _I, _I]
        lib.nc_host_read_gbps.restype = ctypes.c_double
        lib.nc_host_math.argtypes = [ctypes.c_int, _P, _P, _I]
        _LIB = lib
    return _LIB


def _ptr(a):
    return None if a is None else a.ctypes.data


def set_threads(n: int) -> int:
    return load().nc_host_set_threads(n)


def isa() -> str:
    return ISA_NAMES[load().nc_host_isa()]


def limit_isa(limit: int) -> str:
    return ISA_NAMES[load().nc_host_limit_isa(limit)]


def matmul_i8_token(xq, xs, q, scales, bias=None, residual=None) -> np.ndarray:
    xq, q = np.ascontiguousarray(xq, np.int8), np.ascontiguousarray(q, np.int8)
    xs, scales = np.ascontiguousarray(xs, np.float32), np.ascontiguousarray(scales, np.float32)
    bias = None if bias is None else np.ascontiguousarray(bias, np.float32)
    residual = None if residual is None else np.ascontiguousarray(residual, np.float32)
    m, k = xq.shape
    n = q.shape[0]
    y = np.empty((m, n), np.float32)
    load().nc_host_matmul_i8_token(_ptr(y), _ptr(xq), _ptr(xs), _ptr(q), _ptr(scales), _ptr(bias), _ptr(residual),
                                   m, n, k)
    return y


def matmul_i8_token_acc(xq, q) -> np.ndarray:
    xq, q = np.ascontiguousarray(xq, np.int8), np.ascontiguousarray(q, np.int8)
    m, k = xq.shape
    acc = np.empty((m, q.shape[0]), np.int32)
    load().nc_host_matmul_i8_token_acc(_ptr(acc), _ptr(xq), _ptr(q), m, q.shape[0], k)
    return acc


def time_matmul_i8_token(xq, xs, q_copies, ws_copies, reps: int) -> float:
    """Seconds for ``reps`` passes over the stacked weight copies ``[copies, N, K]``."""
    copies, n, k = q_copies.shape
    m = xq.shape[0]
    y = np.empty((m, n), np.float32)
    return load().nc_host_time_matmul_i8_token(_ptr(y), _ptr(xq), _ptr(xs), _ptr(q_copies), _ptr(ws_copies),
                                               m, n, k, copies, reps)


def read_gbps(nbytes: int = 1 << 30, reps: int = 3) -> float:
    buf = np.ones(nbytes // 8, np.int64)
    return load().nc_host_read_gbps(_ptr(buf), buf.nbytes, reps)


MATH_KINDS = {"nc_exp": 0, "nc_sin": 1, "nc_cos": 2, "exp": 3, "sin": 4, "cos": 5}


def math(kind: str, x) -> np.ndarray:
    """Elementwise nc_expf/nc_sinf/nc_cosf (the shared GPU/host functions) or libm's expf/sinf/cosf."""
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    load().nc_host_math(MATH_KINDS[kind], _ptr(out), _ptr(x), x.size)
    return out


def _sig(name, n_ptr, n_int, extra=()):
    fn = getattr(load(), name)
    fn.argtypes = [_P] * n_ptr + [_I] * n_int + list(extra)
    return fn


def softmax_causal(s, past: int) -> np.ndarray:
    """softmax(s + causal mask) over rows of s[heads, seq, past + seq], in the GPU kernel's order."""
    s = np.ascontiguousarray(s, np.float32)
    heads, seq, _ = s.shape
    y = np.empty_like(s)
    _sig("nc_host_softmax_causal", 2, 3)(_ptr(y), _ptr(s), heads, seq, past)
    return y


def rope(x, inv_freq, past: int) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    heads, seq, d = x.shape
    y = np.empty_like(x)
    _sig("nc_host_rope", 3, 4)(_ptr(y), _ptr(x), _ptr(np.ascontiguousarray(inv_freq, np.float32)), heads, seq, d, past)
    return y


def silu_mul(g, u) -> np.ndarray:
    g, u = np.ascontiguousarray(g, np.float32), np.ascontiguousarray(u, np.float32)
    y = np.empty_like(g)
    _sig("nc_host_silu_mul", 3, 1)(_ptr(y), _ptr(g), _ptr(u), g.size)
    return y


def rms_norm_quant(x, gamma, eps: float):
    x = np.ascontiguousarray(x, np.float32)
    m, k = x.shape
    normed, xq, xs = np.empty_like(x), np.empty((m, k), np.int8), np.empty(m, np.float32)
    _sig("nc_host_rms_norm_quant", 5, 2, [ctypes.c_float])(_ptr(normed), _ptr(xq), _ptr(xs), _ptr(x),
                                                            _ptr(np.ascontiguousarray(gamma, np.float32)), m, k, eps)
    return normed, xq, xs


def rms_norm_quant_pool(x, gamma, eps: float):
    """``rms_norm_quant`` with the rows spread over the host pool (the same bits)."""
    x = np.ascontiguousarray(x, np.float32)
    m, k = x.shape
    normed, xq, xs = np.empty_like(x), np.empty((m, k), np.int8), np.empty(m, np.float32)
    _sig("nc_host_rms_norm_quant_pool", 5, 2, [ctypes.c_float])(
        _ptr(normed), _ptr(xq), _ptr(xs), _ptr(x), _ptr(np.ascontiguousarray(gamma, np.float32)), m, k, eps)
    return normed, xq, xs


def rope_append_attention(qkv, kcache, vcache, inv_freq, heads: int, kv: int, d: int, past: int, scale: float):
    """RoPE + cache append (in place on qkv and the caches), then attention; returns the context."""
    m = qkv.shape[0]
    cap = kcache.shape[1]
    inv_freq = np.ascontiguousarray(inv_freq, np.float32)
    _sig("nc_host_rope_append", 4, 6)(_ptr(qkv), _ptr(kcache), _ptr(vcache), _ptr(inv_freq), m, heads, kv, d,
                                      past, cap)
    ctx = np.empty((m, heads * d), np.float32)
    _sig("nc_host_attention", 4, 6, [ctypes.c_float])(_ptr(ctx), _ptr(qkv), _ptr(kcache), _ptr(vcache), m, heads,
                                                       kv, d, past, cap, scale)
    return ctx


def matmul_i8_token_swiglu(xq, xs, qg, sg, qu, su) -> np.ndarray:
    m, k = xq.shape
    n = qg.shape[0]
    h = np.empty((m, n), np.float32)
    args = [np.ascontiguousarray(a) for a in (xq, xs, qg, sg, qu, su)]
    _sig("nc_host_matmul_i8_token_swiglu", 7, 3)(_ptr(h), *[_ptr(a) for a in args], m, n, k)
    return h


def matmul_i8_f32(x, q, scales) -> np.ndarray:
    """The reference's matmul_i8 (float activations) in its 32-chain FMA order (lower.py:294-356)."""
    x, q, scales = (np.ascontiguousarray(a) for a in (x, q, scales))
    m, k = x.shape
    y = np.empty((m, q.shape[0]), np.float32)
    _sig("nc_host_matmul_i8_f32", 4, 3)(_ptr(y), _ptr(x), _ptr(q), _ptr(scales), m, q.shape[0], k)
    return y


def matmul_i8_vnni(xq, xs, offset, q, scales, block: int = 32) -> np.ndarray:
    """The reference's matmul_i8_vnni in its Dp4 / block-scale order (lower.py:359-397)."""
    xq, xs, offset, q, scales = (np.ascontiguousarray(a) for a in (xq, xs, offset, q, scales))
    m, k = xq.shape
    y = np.empty((m, q.shape[0]), np.float32)
    _sig("nc_host_matmul_i8_vnni", 6, 4)(_ptr(y), _ptr(xq), _ptr(xs), _ptr(offset), _ptr(q), _ptr(scales), m,
                                         q.shape[0], k, block)
    return y
