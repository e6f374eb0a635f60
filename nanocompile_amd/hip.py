"""The HIP library over ctypes: loading, device memory, and the kernel calling convention.

Every kernel entry point has the reference's generated-kernel signature
(codegen_c.py:5-10, 254):

    int32_t nc_name(void **p, const int64_t *s);

``p`` holds device pointers (output first), ``s`` the sizes. A non-zero return
is a rejected call (2), a refused launch (3) or, from :func:`sync`, a kernel
that reported bad input (1, the reference's gather bounds check). Each becomes
a :class:`KernelError`, as the reference's runtime does (runtime.py:298-318).

Nothing here falls back to the CPU. If the library is not built, or there is
no GPU, the first call raises.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

from nanocompile_amd.build import LIBRARY

NC_OK, NC_FAIL_INDEX, NC_BAD_ARGS, NC_LAUNCH_FAILED = 0, 1, 2, 3


class KernelError(RuntimeError):
    """A kernel rejected its input, or the runtime refused a launch."""


class LibraryMissing(RuntimeError):
    """The HIP library is not built (run ``__graft_entry__.build()``)."""


_LIB: ctypes.CDLL | None = None
_DEVICE: int | None = None
_KERNEL_ARGS = [ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(ctypes.c_int64)]

# Exported functions that are not kernels, with their ctypes signatures.
_RUNTIME = {
    "nc_last_error": (ctypes.c_char_p, []),
    "nc_device_count": (ctypes.c_int32, []),
    "nc_init": (ctypes.c_int32, [ctypes.c_int32]),
    "nc_device_info": (ctypes.c_int32, [ctypes.c_char_p, ctypes.c_int64] + [ctypes.POINTER(ctypes.c_int64)] * 4),
    "nc_runtime_version": (ctypes.c_int32, [ctypes.POINTER(ctypes.c_int64)] * 2),
    "nc_library_digest": (ctypes.c_char_p, []),
    "nc_schedule_info": (ctypes.c_int32, [ctypes.c_int32, ctypes.POINTER(ctypes.c_int64)]),
    "nc_decode_schedule_info": (ctypes.c_int32, [ctypes.c_int64] * 3 + [ctypes.POINTER(ctypes.c_int64)]),
    "nc_attention_schedule_info": (ctypes.c_int32, [ctypes.c_int64, ctypes.POINTER(ctypes.c_int64)]),
    "nc_malloc": (ctypes.c_void_p, [ctypes.c_int64]),
    "nc_free": (ctypes.c_int32, [ctypes.c_void_p]),
    "nc_host_malloc": (ctypes.c_void_p, [ctypes.c_int64]),
    "nc_host_free": (ctypes.c_int32, [ctypes.c_void_p]),
    "nc_memcpy_h2d": (ctypes.c_int32, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]),
    "nc_memcpy_d2h": (ctypes.c_int32, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]),
    "nc_memcpy_h2d_async": (ctypes.c_int32, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]),
    "nc_memcpy_d2h_async": (ctypes.c_int32, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]),
    "nc_memcpy_d2d": (ctypes.c_int32, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]),
    "nc_memcpy_rows": (ctypes.c_int32, [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int64,
                                        ctypes.c_int64, ctypes.c_int64, ctypes.c_int32]),
    "nc_sync": (ctypes.c_int32, []),
    "nc_stream_handle": (ctypes.c_void_p, []),
    "nc_error_word": (ctypes.c_void_p, []),
    "nc_event_create": (ctypes.c_void_p, []),
    "nc_event_record": (ctypes.c_int32, [ctypes.c_void_p]),
    "nc_event_elapsed_ms": (ctypes.c_int32, [ctypes.c_void_p, ctypes.c_void_p, ctypes.POINTER(ctypes.c_float)]),
    "nc_event_destroy": (ctypes.c_int32, [ctypes.c_void_p]),
    "nc_capture_begin": (ctypes.c_int32, []),
    "nc_capture_end": (ctypes.c_int32, [ctypes.POINTER(ctypes.c_void_p)]),
    "nc_graph_launch": (ctypes.c_int32, [ctypes.c_void_p]),
    "nc_graph_destroy": (ctypes.c_int32, [ctypes.c_void_p]),
}


def load(path: Path | str = LIBRARY) -> ctypes.CDLL:
    """The library, loaded once. Loading does not touch the GPU."""
    global _LIB
    if _LIB is None:
        path = Path(path)
        if not path.exists():
            raise LibraryMissing(f"{path} is not built; run __graft_entry__.build()")
        lib = ctypes.CDLL(str(path))
        for name, (restype, argtypes) in _RUNTIME.items():
            fn = getattr(lib, name)
            fn.restype, fn.argtypes = restype, argtypes
        _LIB = lib
    return _LIB


def last_error() -> str:
    return load().nc_last_error().decode(errors="replace")


def _check(status: int, what: str) -> None:
    if status != NC_OK:
        raise KernelError(f"{what} failed with {status}: {last_error()}")


def init(device: int = 0) -> None:
    """Bind the library to ``device`` (once per process)."""
    global _DEVICE
    if _DEVICE == device:
        return
    lib = load()
    if lib.nc_device_count() <= device:
        raise KernelError(f"no HIP device {device}: the GPU path needs a GPU")
    _check(lib.nc_init(device), "nc_init")
    _DEVICE = device


def device_info() -> dict:
    init()
    name = ctypes.create_string_buffer(64)
    cus, lds, hbm, clock = (ctypes.c_int64() for _ in range(4))
    _check(load().nc_device_info(name, 64, ctypes.byref(cus), ctypes.byref(lds), ctypes.byref(hbm),
                                 ctypes.byref(clock)), "nc_device_info")
    return {"arch": name.value.decode(), "compute_units": cus.value, "lds_bytes": lds.value,
            "hbm_bytes": hbm.value, "clock_khz": clock.value}


def runtime_version() -> tuple[int, int]:
    """(HIP runtime version, driver version)."""
    init()
    runtime, driver = ctypes.c_int64(), ctypes.c_int64()
    _check(load().nc_runtime_version(ctypes.byref(runtime), ctypes.byref(driver)), "nc_runtime_version")
    return runtime.value, driver.value


def library_digest() -> str:
    """The hash of the sources and flags the loaded library was built from (no GPU needed)."""
    return load().nc_library_digest().decode()


def schedule_info(schedule: int) -> dict | None:
    """The launch shape of projection schedule ``schedule`` (a table lookup; no GPU needed)."""
    out = (ctypes.c_int64 * 16)()
    if load().nc_schedule_info(int(schedule), out) != NC_OK:
        return None
    if out[0] == 0:
        return {"schedule": int(schedule), "kernel": "gemv", "lanes_per_row": out[1], "waves": out[2],
                "load_bytes": out[3]}
    return {"schedule": int(schedule), "kernel": "mfma", "tile_m": out[1], "tile_n": out[2], "k_stage": out[3],
            "wave_m": out[4], "wave_n": out[5], "stages": out[6], "threads": out[7], "lds_bytes": out[8],
            "lds_bytes_pair": out[9]}


def decode_schedule_info(k: int, kind: int, schedule: int) -> dict | None:
    """A decode projection schedule's launch shape (a table lookup; no GPU needed), or None."""
    out = (ctypes.c_int64 * 4)()
    if load().nc_decode_schedule_info(int(k), int(kind), int(schedule), out) != NC_OK:
        return None
    return {"lanes_per_row": out[0], "waves": out[1], "load_bytes": out[2]}


def attention_schedule_info(schedule: int) -> int | None:
    """Query rows a prefill attention workgroup takes under ``schedule`` (no GPU needed), or None."""
    out = (ctypes.c_int64 * 2)()
    if load().nc_attention_schedule_info(int(schedule), out) != NC_OK:
        return None
    return int(out[0])


def kernel(name: str):
    """The entry point ``name`` with the kernel calling convention."""
    fn = getattr(load(), name)
    fn.restype, fn.argtypes = ctypes.c_int32, _KERNEL_ARGS
    return fn


PAD = 16   # entries every p[] and s[] array carries: optional trailing operands read NULL / 0


def call(name: str, pointers, sizes) -> None:
    """Enqueue kernel ``name`` on the library stream; raises on a rejected launch.

    The arrays are padded with NULL pointers and zero sizes to ``PAD``
    entries, so an entry point's optional trailing operands (a position read
    from the device, say) are NULL unless the caller gives them.
    """
    init()
    p = (ctypes.c_void_p * max(PAD, len(pointers)))(*[_address(x) for x in pointers])
    s = (ctypes.c_int64 * max(PAD, len(sizes)))(*[int(v) for v in sizes])
    status = kernel(name)(p, s)
    if status != NC_OK:
        raise KernelError(f"{name} failed with {status}: {last_error()}")


def sync() -> None:
    """Wait for the stream; a kernel's failure code becomes a KernelError."""
    status = load().nc_sync()
    if status == NC_FAIL_INDEX:
        raise KernelError("a gather index is out of range")
    if status != NC_OK:
        raise KernelError(f"a kernel failed with {status}: {last_error()}")


def _address(x) -> int | None:
    if x is None:
        return None
    if isinstance(x, int):
        return x
    return x.ptr


_ALLOCATIONS = 0


def allocations() -> int:
    """How many device allocations this process's DeviceArrays have made (each one ``hipMalloc``)."""
    return _ALLOCATIONS


def copy_rows(dst: int, dst_pitch: int, src: int, src_pitch: int, width: int, height: int,
              to_device: bool) -> None:
    """``height`` rows of ``width`` bytes between host and device memory, each side with its own
    pitch (bytes from one row's start to the next's); waits for the copy."""
    if width <= 0 or height <= 0:
        return
    if width > dst_pitch or width > src_pitch:
        raise ValueError(f"rows of {width} bytes do not fit pitches {dst_pitch} / {src_pitch}")
    _check(load().nc_memcpy_rows(dst, dst_pitch, src, src_pitch, width, height, 1 if to_device else 2),
           "nc_memcpy_rows")


class DeviceArray:
    """A device allocation with a dtype and shape. Freed when dropped, unless it is a view."""

    __slots__ = ("ptr", "shape", "dtype", "nbytes", "_owner", "__weakref__")

    def __init__(self, shape, dtype, ptr: int | None = None, owner=None) -> None:
        init()
        self.shape = tuple(int(d) for d in shape)
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        if ptr is None:
            global _ALLOCATIONS
            ptr = load().nc_malloc(max(self.nbytes, 1))
            if not ptr:
                raise MemoryError(f"nc_malloc({self.nbytes}) failed: {last_error()}")
            _ALLOCATIONS += 1
            owner = True
        self.ptr = int(ptr)
        self._owner = owner

    @classmethod
    def from_host(cls, array: np.ndarray) -> "DeviceArray":
        array = np.ascontiguousarray(array)
        out = cls(array.shape, array.dtype)
        out.upload(array)
        return out

    def upload(self, array: np.ndarray) -> None:
        array = np.ascontiguousarray(array, dtype=self.dtype)
        if array.nbytes != self.nbytes:
            raise ValueError(f"upload of {array.nbytes} bytes into {self.nbytes}")
        if self.nbytes:
            _check(load().nc_memcpy_h2d(self.ptr, array.ctypes.data, self.nbytes), "nc_memcpy_h2d")

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, dtype=self.dtype)
        if self.nbytes:
            _check(load().nc_memcpy_d2h(out.ctypes.data, self.ptr, self.nbytes), "nc_memcpy_d2h")
        return out

    def view(self, shape, dtype=None, offset_bytes: int = 0) -> "DeviceArray":
        """A view of part of this allocation; keeps the allocation alive."""
        dtype = np.dtype(dtype or self.dtype)
        nbytes = int(np.prod(shape, dtype=np.int64)) * dtype.itemsize
        if offset_bytes < 0 or offset_bytes + nbytes > self.nbytes:
            raise ValueError("view outside its allocation")
        return DeviceArray(shape, dtype, self.ptr + offset_bytes, owner=self)

    def __del__(self) -> None:
        if getattr(self, "_owner", None) is True and _LIB is not None:
            _LIB.nc_free(self.ptr)
            self._owner = None

    def __repr__(self) -> str:
        return f"<DeviceArray {self.dtype}{list(self.shape)} at {self.ptr:#x}>"


class Event:
    """A HIP event on the library stream, for timing kernels where they run."""

    def __init__(self) -> None:
        init()
        self.handle = load().nc_event_create()
        if not self.handle:
            raise KernelError(f"nc_event_create failed: {last_error()}")

    def record(self) -> None:
        _check(load().nc_event_record(self.handle), "nc_event_record")

    def elapsed_ms(self, later: "Event") -> float:
        ms = ctypes.c_float()
        _check(load().nc_event_elapsed_ms(self.handle, later.handle, ctypes.byref(ms)), "nc_event_elapsed_ms")
        return float(ms.value)

    def __del__(self) -> None:
        if getattr(self, "handle", None) and _LIB is not None:
            _LIB.nc_event_destroy(self.handle)


class Graph:
    """Launches captured from the library stream, replayed as one HIP graph."""

    def __init__(self, handle: int) -> None:
        self.handle = handle

    @classmethod
    def capture(cls, fn) -> "Graph":
        init()
        _check(load().nc_capture_begin(), "nc_capture_begin")
        try:
            fn()
        finally:
            out = ctypes.c_void_p()
            status = load().nc_capture_end(ctypes.byref(out))
        _check(status, "nc_capture_end")
        return cls(out.value)

    def launch(self) -> None:
        _check(load().nc_graph_launch(self.handle), "nc_graph_launch")

    def __del__(self) -> None:
        if getattr(self, "handle", None) and _LIB is not None:
            _LIB.nc_graph_destroy(self.handle)
