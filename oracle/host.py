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
