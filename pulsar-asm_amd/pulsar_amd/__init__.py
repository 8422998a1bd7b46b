"""pulsar_amd -- Python view of the gfx950 C ABI (include/pulsar_amd.h).

The compute path is libpulsar_amd.so, built in-tree by build.py. Loading
fails loudly when the library is missing: there is no CPU or eager fallback.
torch is used only for device memory and streams (tensors are passed to the C
ABI as raw pointers).
"""
import ctypes as C
import os

from . import _abi

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "libpulsar_amd.so")

_lib = None


def lib():
    """The loaded C ABI (raises if the HIP library has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with python pulsar-asm_amd/pulsar_amd/build.py "
                               "(there is no fallback path)")
        _lib = _abi.bind(C.CDLL(LIB_PATH))
    return _lib


class PQError(RuntimeError):
    pass


def check(rc, what=""):
    if rc != 0:
        msg = lib().pq_last_error().decode(errors="replace")
        raise PQError(f"{what} failed ({rc}): {msg}")
    return rc


from .ops import *  # noqa: E402,F401,F403
