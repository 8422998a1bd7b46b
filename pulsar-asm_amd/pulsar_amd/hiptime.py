"""HIP events for timing launches on a given stream (ctypes over libamdhip64).

Events are created with hipEventDisableSystemFence so recording one does not
add a system-scope memory fence to the stream: the elapsed time between an
event recorded before a launch and one recorded after it then tracks the
kernel's own duration (what rocprofv3's kernel trace reports) instead of the
fence's cost.
"""
import ctypes as C

_hip = None
HIP_EVENT_DISABLE_SYSTEM_FENCE = 0x20000000


def _lib():
    global _hip
    if _hip is None:
        _hip = C.CDLL("libamdhip64.so")
        _hip.hipEventCreateWithFlags.argtypes = [C.POINTER(C.c_void_p), C.c_uint]
        _hip.hipEventRecord.argtypes = [C.c_void_p, C.c_void_p]
        _hip.hipEventSynchronize.argtypes = [C.c_void_p]
        _hip.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), C.c_void_p, C.c_void_p]
        _hip.hipEventDestroy.argtypes = [C.c_void_p]
    return _hip


class Event:
    def __init__(self):
        self.h = C.c_void_p()
        rc = _lib().hipEventCreateWithFlags(C.byref(self.h), HIP_EVENT_DISABLE_SYSTEM_FENCE)
        if rc != 0:
            raise RuntimeError(f"hipEventCreateWithFlags failed ({rc})")

    def record(self, stream):
        rc = _lib().hipEventRecord(self.h, C.c_void_p(stream))
        if rc != 0:
            raise RuntimeError(f"hipEventRecord failed ({rc})")

    def synchronize(self):
        _lib().hipEventSynchronize(self.h)

    def elapsed_ms(self, end):
        ms = C.c_float()
        rc = _lib().hipEventElapsedTime(C.byref(ms), self.h, end.h)
        if rc != 0:
            raise RuntimeError(f"hipEventElapsedTime failed ({rc})")
        return ms.value

    def __del__(self):
        if self.h and _hip is not None:
            _hip.hipEventDestroy(self.h)
            self.h = None
