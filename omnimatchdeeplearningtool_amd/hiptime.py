"""HIP event timing on the library stream (ctypes over libamdhip64).

torch.cuda.Event only sees torch's current stream; libomhip enqueues on its
own stream, so the bench records hipEvents on that stream directly.
"""
from __future__ import annotations

import ctypes
import ctypes.util
import os

_HIP = None


def _hip():
    global _HIP
    if _HIP is None:
        for cand in ("/opt/rocm/lib/libamdhip64.so", ctypes.util.find_library("amdhip64") or "libamdhip64.so"):
            try:
                _HIP = ctypes.CDLL(cand)
                break
            except OSError:
                continue
        if _HIP is None:
            raise RuntimeError("libamdhip64.so not found")
        _HIP.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        _HIP.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        _HIP.hipEventSynchronize.argtypes = [ctypes.c_void_p]
        _HIP.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        _HIP.hipEventDestroy.argtypes = [ctypes.c_void_p]
    return _HIP


class StreamTimer:
    """Brackets work enqueued on `stream` with two hipEvents; .ms() waits and returns elapsed ms."""

    def __init__(self, stream: int):
        h = _hip()
        self.stream = ctypes.c_void_p(stream)
        self.e0, self.e1 = ctypes.c_void_p(), ctypes.c_void_p()
        assert h.hipEventCreate(ctypes.byref(self.e0)) == 0
        assert h.hipEventCreate(ctypes.byref(self.e1)) == 0

    def start(self):
        assert _hip().hipEventRecord(self.e0, self.stream) == 0

    def stop(self):
        assert _hip().hipEventRecord(self.e1, self.stream) == 0

    def ms(self) -> float:
        h = _hip()
        assert h.hipEventSynchronize(self.e1) == 0
        t = ctypes.c_float()
        assert h.hipEventElapsedTime(ctypes.byref(t), self.e0, self.e1) == 0
        return float(t.value)

    def __del__(self):
        try:
            h = _hip()
            h.hipEventDestroy(self.e0)
            h.hipEventDestroy(self.e1)
        except Exception:
            pass
