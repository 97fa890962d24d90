"""Kernel-level timing with HIP events recorded by the dispatch itself.

``eg_time_kernel`` arms the next entry-point call so that one of its kernels is
launched with hipExtLaunchKernelGGL and a pair of events; the events are
stamped at that kernel's start and end on the stream it runs on. This measures
the kernel alone: no host launch latency and no gap between an event and the
kernel that follows it lands in the figure (a separately recorded
torch.cuda.Event pair adds several microseconds to every region).

The events come from the HIP runtime torch has already loaded (same soname as
the library's own dependency), through ctypes.
"""

from __future__ import annotations

import ctypes

import torch  # noqa: F401  (loads the HIP runtime first)

from . import _lib

_hip = None


def _runtime():
    global _hip
    if _hip is None:
        h = ctypes.CDLL("libamdhip64.so.7")
        h.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        h.hipEventCreate.restype = ctypes.c_int
        h.hipEventDestroy.argtypes = [ctypes.c_void_p]
        h.hipEventDestroy.restype = ctypes.c_int
        h.hipEventSynchronize.argtypes = [ctypes.c_void_p]
        h.hipEventSynchronize.restype = ctypes.c_int
        h.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p,
                                          ctypes.c_void_p]
        h.hipEventElapsedTime.restype = ctypes.c_int
        _hip = h
    return _hip


class KernelTimer:
    """A reusable start/stop event pair for timing one kernel launch."""

    def __init__(self):
        h = _runtime()
        self.start = ctypes.c_void_p()
        self.stop = ctypes.c_void_p()
        for ev in (self.start, self.stop):
            rc = h.hipEventCreate(ctypes.byref(ev))
            if rc != 0:
                raise RuntimeError(f"hipEventCreate failed ({rc})")

    def arm(self, index: int) -> None:
        """Time kernel number ``index`` of this thread's launches, counted from the
        next library call on (across the calls that follow it)."""
        _lib.call("eg_time_kernel", self.start, self.stop, int(index))

    def label(self) -> str:
        """Name of the kernel the last arm launched ("" before that launch)."""
        raw = _lib.query("eg_time_kernel_label")
        return raw.decode() if raw else ""

    def fired(self) -> bool:
        """Whether the armed launch has run (drops the arm either way)."""
        return not _lib.query("eg_time_kernel_missed")

    def elapsed_ms(self) -> float:
        if _lib.query("eg_time_kernel_missed"):
            raise RuntimeError("the armed kernel launch did not run")
        h = _runtime()
        rc = h.hipEventSynchronize(self.stop)
        if rc != 0:
            raise RuntimeError(f"hipEventSynchronize failed ({rc})")
        ms = ctypes.c_float()
        rc = h.hipEventElapsedTime(ctypes.byref(ms), self.start, self.stop)
        if rc != 0:
            raise RuntimeError(f"hipEventElapsedTime failed ({rc}): the armed kernel did not run")
        return float(ms.value)

    def close(self) -> None:
        h = _runtime()
        for ev in (self.start, self.stop):
            if ev.value:
                h.hipEventDestroy(ev)
                ev.value = None

    def __del__(self):  # pragma: no cover
        try:
            self.close()
        except Exception:
            pass
