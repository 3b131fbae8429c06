"""Loader and ctypes signatures of libbmo_attn.so."""
from __future__ import annotations

import ctypes
import os
import re
import subprocess

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG_DIR)
LIB_PATH = os.path.join(PKG_DIR, "libbmo_attn.so")
HEADER = os.path.join(ROOT, "include", "bmo_attn.h")
CSRC = os.path.join(PKG_DIR, "csrc")

_lib = None

P = ctypes.c_void_p
i32 = ctypes.c_int
i64 = ctypes.c_int64
f32 = ctypes.c_float

SIGNATURES = {
    "bmo_kv_ring_stripe_bytes": (i64, [i32, i32]),
    "bmo_kv_ring_create": (P, [i32, i32, i32, i32, i32]),
    "bmo_kv_ring_free": (None, [P]),
    "bmo_kv_ring_geometry": (i32, [P, P, P, P, P, P]),
    "bmo_kv_ring_bytes": (i64, [P]),
    "bmo_kv_ring_k_base": (P, [P]),
    "bmo_kv_ring_v_base": (P, [P]),
    "bmo_kv_ring_reset": (i32, [P, i32, P]),
    "bmo_kv_ring_last_error": (ctypes.c_char_p, [P]),
    "bmo_kv_ring_append": (i32, [P, i32, i32, P, P, P, P, P]),
    "bmo_kv_ring_decode": (i32, [P, i32, i32, P, P, i32, P, P, f32, P]),
    "bmo_kv_ring_append_decode": (i32, [P, i32, i32, P, P, i32, P, P, P, P, f32, P]),
    "bmo_kv_ring_append_decode_rope": (i32, [P, i32, i32, P, P, i32, P, P, P, P, f32, f32, P]),
    "bmo_launch_gemv_q4_0_q8_1": (i32, [P, P, P, i32, i32, P, P]),
    "bmo_positions_advance": (i32, [P, i32, i32, P]),
    "bmo_kv_ring_write": (i32, [P, i32, i32, i64, i32, P, P, P]),
    "bmo_kv_ring_prefill": (i32, [P, i32, i32, P, P, i32, i32, P, P, P, P, f32, P]),
    "bmo_kv_ring_prefill_noalloc": (i32, [P, i32, i32, P, P, i32, i32, P, P, P, P, f32, P]),
    "bmo_kv_ring_copy_k_f32": (i32, [P, i32, i32, i32, i32, P, i32]),
    "bmo_kv_ring_export_q4_0": (i64, [P, i32, i32, i32, i32, i32, P, i64]),
    "bmo_kv_ring_import_q4_0": (i64, [P, i32, i32, i32, i32, i32, P, i64]),
    "bmo_launch_decode_attention": (None, [P, P, P, P, P, P, i32, i32, i32, i32, i32, i32, P, P]),
    "bmo_attn_session_create": (P, [P, i32, i32, f32, f32]),
    "bmo_attn_session_free": (None, [P]),
    "bmo_attn_session_reset": (i32, [P]),
    "bmo_attn_session_pos": (i64, [P]),
    "bmo_attn_session_stream": (P, [P]),
    "bmo_attn_session_forward": (i32, [P, i32, P, P, P, P]),
    "bmo_attn_session_capture": (i32, [P, P, P, P, P]),
    "bmo_attn_session_has_graph": (i32, [P]),
    "bmo_attn_session_replay": (i32, [P, i32]),
    "bmo_attn_session_last_error": (ctypes.c_char_p, [P]),
    "bmo_attn_session_begin_step": (i32, [P, i32]),
    "bmo_attn_session_layer": (i32, [P, i32, P, P, P, P]),
    "bmo_attn_session_end_step": (i32, [P]),
    "bmo_attn_session_reset_async": (i32, [P]),
    "bmo_attn_session_sync": (i32, [P]),
    "bmo_attn_session_capture_begin": (i32, [P]),
    "bmo_attn_session_capture_end": (i32, [P]),
}


def build(force: bool = True) -> str:
    """Compile libbmo_attn.so for gfx950 with bmo_jetson_amd/csrc/Makefile."""
    args = ["make", "-C", CSRC, "-j4"]
    if force:
        args.insert(1, "-B")
    subprocess.run(args, check=True, stdout=subprocess.DEVNULL)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    """The loaded library; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.isfile(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it first (make -C {CSRC}); "
                "there is no CPU fallback")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def header_symbols() -> list[str]:
    """Names of every function include/bmo_attn.h declares with BMO_ATTN_API."""
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = "\n".join(l for l in text.splitlines() if not l.lstrip().startswith("#"))
    names = re.findall(r"BMO_ATTN_API\s+[^;(]*?\b(\w+)\s*\(", text)
    return sorted(set(names))
