"""ctypes binding of libbootstrap_hip.so — the Python twin of the engine's P/Invoke layer.

Mirrors ``src/Bootstrap.Engine/Metal.cs``: ``KernelArgs`` (Metal.cs:6-12), the native
table (Metal.cs:14-42), ``GpuBuffer`` (Metal.cs:44-56), ``Binding`` (Metal.cs:58) and the
``Metal`` device wrapper (Metal.cs:60-115) with the same operations and error behaviour:
every failing native call raises ``HipError`` carrying ``boot_error`` (Metal.cs:69).

Device buffers live in HBM, so the host span ``GpuBuffer.Values<T>()`` becomes explicit
``read``/``write`` copies, and ``Grow``'s span copy becomes ``Device.copy``.
There is no CPU fallback: if the library or a gfx950 device is missing, construction fails.
"""
from __future__ import annotations

import ctypes
import os
import weakref
from typing import NamedTuple, Optional

import numpy as np

LIBRARY_NAME = "libbootstrap_hip.so"
_HERE = os.path.dirname(os.path.abspath(__file__))


class HipError(RuntimeError):
    """A native call failed (Metal.cs:69 raises InvalidOperationException)."""


class KernelArgs(ctypes.Structure):
    """64-byte argument block: Metal.cs:6-12 / kernels.metal:6 (struct P)."""

    _fields_ = [(name, ctypes.c_uint32) for name in ("N", "M", "K", "Kind", "Position", "Flags", "A", "B")] + \
               [(name, ctypes.c_float) for name in ("Epsilon", "Theta", "Scale", "Value")] + \
               [(name, ctypes.c_uint32) for name in ("C", "D", "E", "F")]


assert ctypes.sizeof(KernelArgs) == 64

# Exported C ABI (include/bootstrap_hip.h): name -> (restype, argtypes)
_VP, _CP, _U64, _I, _U32 = ctypes.c_void_p, ctypes.c_char_p, ctypes.c_uint64, ctypes.c_int, ctypes.c_uint32
SIGNATURES = {
    "boot_create": (_VP, [_CP]),
    "boot_error": (_CP, [_VP]),
    "boot_destroy": (None, [_VP]),
    "boot_buffer": (_VP, [_VP, _U64]),
    "boot_map": (_VP, [_VP, _CP]),
    "boot_contents": (_VP, [_VP]),
    "boot_release_buffer": (None, [_VP]),
    "boot_allocated": (_U64, [_VP]),
    "boot_begin": (_I, [_VP]),
    "boot_clear": (_I, [_VP, _VP]),
    "boot_dispatch": (_I, [_VP, _CP, ctypes.POINTER(_VP), ctypes.POINTER(_U64), _I, _VP, _I,
                           _U32, _U32, _U32, _U32, _U32, _U32, _VP, _U64]),
    "boot_dispatch_noalloc": (_I, [_VP, _CP, ctypes.POINTER(_VP), ctypes.POINTER(_U64), _I, _VP, _I,
                                   _U32, _U32, _U32, _U32, _U32, _U32, _VP, _U64]),
    "boot_end": (_I, [_VP]),
    "boot_profile": (None, [_VP, _I]),
    "boot_wall_reset": (_I, [_VP, _I]),
    "boot_wall_read": (None, [_VP, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double)]),
    "boot_kernel_wall_json": (_CP, [_VP]),
    "boot_buffer_size": (_U64, [_VP]),
    "boot_copy": (_I, [_VP, _VP, _U64, _VP, _U64, _U64]),
    "boot_write": (_I, [_VP, _VP, _U64, _VP, _U64]),
    "boot_read": (_I, [_VP, _VP, _U64, _VP, _U64]),
}

_lib: Optional[ctypes.CDLL] = None


def library_path() -> str:
    """In-tree build location (the package directory); BOOTSTRAP_HIP_LIBRARY overrides."""
    return os.environ.get("BOOTSTRAP_HIP_LIBRARY", os.path.join(_HERE, LIBRARY_NAME))


def load_library(path: Optional[str] = None) -> ctypes.CDLL:
    """Loads the shim (Metal.cs:16-24 resolver, renamed bootstrap_metal -> bootstrap_hip)."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    target = path or library_path()
    if not os.path.exists(target):
        raise HipError(f"{LIBRARY_NAME} is not built ({target}); run __graft_entry__.build()")
    lib = ctypes.CDLL(target)
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    if path is None:
        _lib = lib
    return lib


class Binding(NamedTuple):
    """Buffer plus byte offset bound at one kernel index (Metal.cs:58)."""

    buffer: "GpuBuffer"
    offset: int = 0


class GpuBuffer:
    """Device buffer handle (Metal.cs:44-56). Host access is by explicit copies."""

    def __init__(self, device: "Device", handle: int, length: int):
        self.device = device
        self.handle = handle
        self.length = length

    def write(self, data: np.ndarray, offset: int = 0) -> None:
        array = np.ascontiguousarray(data)
        self.device._check(self.device.lib.boot_write(self.device.handle, self.handle, offset,
                                                      array.ctypes.data, array.nbytes))

    def read(self, dtype, count: int, offset: int = 0) -> np.ndarray:
        out = np.empty(count, dtype=dtype)
        if offset + out.nbytes > self.length:
            raise IndexError("read beyond buffer")
        self.device._check(self.device.lib.boot_read(self.device.handle, self.handle, offset,
                                                     out.ctypes.data, out.nbytes))
        return out

    def fill_bytes(self, value: int, offset: int = 0, count: Optional[int] = None) -> None:
        count = self.length - offset if count is None else count
        self.write(np.full(count, value, dtype=np.uint8), offset)

    def at(self, offset: int) -> Binding:
        return Binding(self, offset)

    def dispose(self) -> None:
        """Releases the buffer once. After ``Device.close`` the context has already freed
        every buffer it owned (boot_destroy), so the handle is then only forgotten."""
        if self.handle and self.device.handle:
            self.device.lib.boot_release_buffer(self.handle)
            self.device._live.discard(self)
        self.handle = 0

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.dispose()


class Device:
    """The ``Metal`` class of Metal.cs:60-115 over the HIP shim."""

    def __init__(self, source: Optional[str] = None, library: Optional[str] = None):
        self.lib = load_library(library)
        handle = self.lib.boot_create(source.encode() if source else None)
        if not handle:
            raise HipError("HIP device unavailable or not gfx950 (boot_create returned NULL)")
        self.handle = handle
        self._live = weakref.WeakSet()   # buffers whose handles close() must invalidate

    # Metal.cs:69
    def _check(self, result: int) -> None:
        if result == 0:
            raise HipError(self.lib.boot_error(self.handle).decode())

    @property
    def allocated_bytes(self) -> int:
        return int(self.lib.boot_allocated(self.handle))

    def allocate(self, nbytes: int) -> GpuBuffer:
        """Metal.cs:70-75: zero-filled, at least 4 bytes."""
        nbytes = max(int(nbytes), 4)
        handle = self.lib.boot_buffer(self.handle, nbytes)
        if not handle:
            self._check(0)
        buffer = GpuBuffer(self, handle, nbytes)
        self._live.add(buffer)
        return buffer

    def set_profiling(self, enabled: bool) -> None:
        self.lib.boot_profile(self.handle, 1 if enabled else 0)

    def reset_wall_timing(self, sample_attention: bool = False, all_kernels: bool = False,
                          kernels_exact: bool = False) -> None:
        """Metal.cs:84 (ResetWallTiming). ``kernels_exact`` times each kernel of the path by
        itself, keyed by kernel function, with events stamped by its own dispatch."""
        mode = 3 if kernels_exact else 2 if all_kernels else 1 if sample_attention else 0
        self._check(self.lib.boot_wall_reset(self.handle, mode))

    def read_wall_timing(self) -> dict:
        """Metal.cs:84-92."""
        import json
        wall = (ctypes.c_double * 7)()
        attention = (ctypes.c_double * 6)()
        self.lib.boot_wall_read(self.handle, wall, attention)
        kernels = json.loads(self.lib.boot_kernel_wall_json(self.handle).decode())
        return {"kernels": kernels, "gpu_ms": wall[0] * 1000, "host_encode_ms": wall[1] * 1000,
                "host_commit_ms": wall[2] * 1000, "host_wait_ms": wall[3] * 1000,
                "command_buffers": wall[4], "dispatches": wall[5], "counter_resolve_ms": wall[6] * 1000,
                "attention_qk_ms": attention[0] * 1000, "attention_softmax_ms": attention[1] * 1000,
                "attention_av_ms": attention[2] * 1000, "attention_qk_count": attention[3],
                "attention_softmax_count": attention[4], "attention_av_count": attention[5]}

    def begin(self) -> None:
        self._check(self.lib.boot_begin(self.handle))

    def clear(self, buffer: GpuBuffer) -> None:
        self._check(self.lib.boot_clear(self.handle, buffer.handle))

    def end(self) -> None:
        self._check(self.lib.boot_end(self.handle))

    def copy(self, dst: GpuBuffer, dst_offset: int, src: GpuBuffer, src_offset: int, nbytes: int) -> None:
        self._check(self.lib.boot_copy(self.handle, dst.handle, dst_offset, src.handle, src_offset, nbytes))

    def dispatch(self, kernel: str, args: KernelArgs, threads: int, group: int, *bindings,
                 noalloc: bool = False) -> None:
        """Metal.cs:96-97."""
        self.dispatch2d(kernel, args, threads, 1, group, *bindings, noalloc=noalloc)

    def dispatch2d(self, kernel: str, args: KernelArgs, threads_x: int, threads_y: int, group: int,
                   *bindings, noalloc: bool = False) -> None:
        """Metal.cs:98-104. ``noalloc`` routes through boot_dispatch_noalloc (split-K scratch
        from the library's static device array; no allocation, no timing sample)."""
        count = len(bindings)
        handles = (ctypes.c_void_p * max(count, 1))()
        offsets = (ctypes.c_uint64 * max(count, 1))()
        for i, b in enumerate(bindings):
            if isinstance(b, GpuBuffer):
                b = Binding(b, 0)
            handles[i] = b.buffer.handle
            offsets[i] = b.offset
        entry = self.lib.boot_dispatch_noalloc if noalloc else self.lib.boot_dispatch
        self._check(entry(self.handle, kernel.encode(), handles, offsets, count, ctypes.byref(args),
                          ctypes.sizeof(KernelArgs), threads_x, threads_y, 1, group, 1, 1, None, 0))

    def close(self) -> None:
        """Metal.cs:114. boot_destroy frees the context and every buffer it still owns, so the
        handles of live GpuBuffer objects are invalidated here (a later dispose is a no-op)."""
        if self.handle:
            for buffer in list(self._live):
                buffer.handle = 0
            self._live.clear()
            self.lib.boot_destroy(self.handle)
            self.handle = 0

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
