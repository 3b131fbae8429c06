"""ctypes binding of libbmo_synth.so (include/bmo_synth.h): the seeded
synthetic inputs of the benchmark configurations, generated on the GPU, and
the benchmark's read probe.
Element c of stream `seed` is a splitmix64 + Box-Muller normal; with
``outliers`` it is multiplied by 8 with probability 1% (configurations 3 and
4).  The CPU restatement is the oracle's (test infrastructure); the two agree
bit for bit, so any part of a configuration's inputs can be regenerated on
the host from its seed."""
from __future__ import annotations

import ctypes
import os

from ._lib import PKG_DIR

SYNTH_PATH = os.path.join(PKG_DIR, "libbmo_synth.so")
_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.isfile(SYNTH_PATH):
            raise OSError(f"{SYNTH_PATH} is not built (python -c 'import __graft_entry__ as g; g.build()')")
        L = ctypes.CDLL(SYNTH_PATH)
        L.bmo_synth_fill_normal.restype = ctypes.c_int
        L.bmo_synth_fill_normal.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_uint64,
                                            ctypes.c_uint64, ctypes.c_int, ctypes.c_void_p]
        L.bmo_synth_read_probe.restype = ctypes.c_int
        L.bmo_synth_read_probe.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p]
        _lib = L
    return _lib


def fill_normal(out, seed: int, offset: int = 0, outliers: bool = False, stream=None) -> None:
    """Fills the contiguous fp32 device tensor ``out`` with elements
    offset .. offset + out.numel() - 1 of stream ``seed``."""
    from .ring import _stream
    assert out.is_contiguous() and str(out.dtype) == "torch.float32"
    rc = lib().bmo_synth_fill_normal(out.data_ptr(), out.numel(), seed & (2**64 - 1),
                                     offset & (2**64 - 1), 1 if outliers else 0, _stream(stream))
    if rc != 0:
        raise RuntimeError(f"bmo_synth_fill_normal failed with code {rc}")


def read_probe(ptr: int, nbytes: int, sink, stream=None) -> None:
    """One pass of the read probe over nbytes of device memory at address
    ptr (16-byte aligned, nbytes a multiple of 16); sink is a device tensor
    of at least 1 KiB."""
    from .ring import _stream
    assert sink.is_cuda and sink.numel() * sink.element_size() >= 1024
    rc = lib().bmo_synth_read_probe(ptr, nbytes, sink.data_ptr(), _stream(stream))
    if rc != 0:
        raise RuntimeError(f"bmo_synth_read_probe failed with code {rc}")


_M64 = (1 << 64) - 1


def mix64(x: int) -> int:
    """splitmix64's output function after its golden-ratio increment."""
    x = (x + 0x9E3779B97F4A7C15) & _M64
    x = ((x ^ (x >> 30)) * 0xBF58476D1CE4E5B9) & _M64
    x = ((x ^ (x >> 27)) * 0x94D049BB133111EB) & _M64
    return x ^ (x >> 31)


def words(seed: int, n: int, offset: int = 0) -> list:
    """Word c of stream seed is mix64(seed ^ mix64(c)), for c = offset .. offset + n - 1."""
    return [mix64((seed & _M64) ^ mix64((offset + i) & _M64)) for i in range(n)]


def positions(seed: int, n: int) -> list:
    """The decode configurations' session positions, U[512, 4096): 512 +
    ((word c of stream seed + 5) >> 11) mod 3584."""
    return [512 + (w >> 11) % 3584 for w in words(seed + 5, n)]
