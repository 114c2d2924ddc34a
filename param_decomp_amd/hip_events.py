"""Raw HIP events for timing kernels on the stream they run on.

The HIP entry points are resolved through the handle of `libpd_mi355x.so`, so they
come from the same HIP runtime instance the kernels (and torch's streams) use; a
process can hold more than one libamdhip64 copy (torch ships its own), and events of
one runtime are invalid handles in another.
"""

from __future__ import annotations

import ctypes

_hip = None


def _lib():
    global _hip
    if _hip is None:
        from param_decomp_amd import _lib as L

        _hip = L.load()
        _hip.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        _hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        _hip.hipEventDestroy.argtypes = [ctypes.c_void_p]
        _hip.hipEventSynchronize.argtypes = [ctypes.c_void_p]
        _hip.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    return _hip


def create(n: int) -> list[int]:
    out = []
    for _ in range(n):
        ev = ctypes.c_void_p()
        rc = _lib().hipEventCreate(ctypes.byref(ev))
        if rc != 0:
            raise RuntimeError(f"hipEventCreate failed: {rc}")
        out.append(ev.value)
    return out


def record(ev: int, stream: int) -> None:
    rc = _lib().hipEventRecord(ev, stream)
    if rc != 0:
        raise RuntimeError(f"hipEventRecord failed: {rc}")


def elapsed_ms(a: int, b: int) -> float:
    ms = ctypes.c_float()
    _lib().hipEventSynchronize(b)
    rc = _lib().hipEventElapsedTime(ctypes.byref(ms), a, b)
    if rc != 0:
        raise RuntimeError(f"hipEventElapsedTime failed: {rc}")
    return float(ms.value)


def destroy(events) -> None:
    for ev in events:
        _lib().hipEventDestroy(ev)


def array(events) -> ctypes.Array:
    arr = (ctypes.c_void_p * len(events))()
    for i, e in enumerate(events):
        arr[i] = e
    return arr
