"""bmo_jetson_amd -- MI355X (gfx950) Q4_0 ring KV cache and sliding-window
attention for bmo_jetson's decode path.

The product is the C-ABI library ``libbmo_attn.so`` (declared in
``include/bmo_attn.h``).  This package is its ctypes binding, in the manner of
the reference's ``bmo_engine.py`` (a ctypes wrapper over ``libbmo.so``): the
functions take device pointers (ints, or tensors exposing ``data_ptr()``) and
HIP streams (ints, ``torch.cuda.Stream`` or ``None`` for the null stream).

There is no CPU fallback: importing the package fails if the library has not
been built (``python -c "import __graft_entry__ as g; g.build()"``).
"""
from ._lib import LIB_PATH, lib, header_symbols, build  # noqa: F401
from .ring import (  # noqa: F401
    KVRing,
    RingError,
    Session,
    launch_decode_attention,
    positions_advance,
    gemv_q4_0_q8_1,
    stripe_bytes,
    BLOCK_Q4_0_BYTES,
)

__all__ = [
    "KVRing",
    "RingError",
    "Session",
    "launch_decode_attention",
    "positions_advance",
    "gemv_q4_0_q8_1",
    "stripe_bytes",
    "BLOCK_Q4_0_BYTES",
    "lib",
    "build",
    "LIB_PATH",
    "header_symbols",
]
